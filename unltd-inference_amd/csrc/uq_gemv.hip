// Decode GEMV kernels for gfx950 (bandwidth-bound, no MFMA).
//
// gemv_kernel      gemv_quant semantics (quants.rs:422-466): y = W x, f32
//                  result of the exact dequantized weights times f32 x.
// gemv_q8k_kernel  gemv_quant_q8k (quants.rs:474-515), bit-exact: x is
//                  quantized to Q8_K in the workgroup, each block's eight
//                  i32 lanes come from integer dots, and the f32 epilogue
//                  replays the reference's operation order per row.
//
// Common structure: a workgroup of 4 waves prepares the activations in LDS
// once; each wave then walks rows (stride = all waves of the grid). In a
// row every lane owns the same 64-weight task (uq_policies.h), so its
// activation data is read from LDS once and stays in VGPRs while the next
// row's weights are prefetched with 128-bit loads. Row sums are reduced
// across the wave with DPP.
//
// Q4_K / Q6_K rows mostly run the streaming forms, in which each wave moves
// its rows into its own LDS ring with coalesced direct-to-LDS nontemporal
// loads and its lanes read their tasks from there:
//   gemv_stream_kernel      K <= 4096 (and the fused gate/up pair)
//   gemv_stream_ks_kernel   4096 < K <= 20480, rows split into 16-block
//                           slices over the waves of a workgroup
//   gemv_q8k_stream_kernel  gemv_quant_q8k, K <= 12288
//   gemv_q8k_ks_kernel      gemv_quant_q8k, one tensor, 4096 < K <= 20480
#include <map>
#include <type_traits>
#include <mutex>

#include "uq_device.h"
#include "uq_internal.h"
#include "uq_policies.h"

namespace uq {

namespace {

constexpr int WAVES = 4;
constexpr int TPB = 64 * WAVES;

int num_cus() {
    static int n = 0;
    if (!n) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            n = v;
        else
            n = 256;
    }
    return n;
}

// ---------------------------- gemv_quant -----------------------------------

template <class F>
__device__ inline XLayout x_layout_at(uint8_t *lds, int K) {
    XLayout L;
    L.NT = round_tasks(F::ntasks(K));
    size_t o = 0;
    L.gsum = (double *)(lds + o);  // 8-byte aligned first
    o += (size_t)(K / 32) * 8;
    L.xq = (uint32_t *)(lds + o);
    o += (size_t)L.NT * 256;
    L.aux = (int *)(lds + o);
    o += F::kAux ? (size_t)L.NT * 32 : 0;
    L.scale = (float *)(lds + o);
    return L;
}

// Register budget: the single GEMV kernels that keep x in VGPRs run NW/4
// waves per SIMD (one workgroup of NW waves per CU), so the allocator is held
// to 512/(NW/4) VGPRs; the gate/up pair (twice the weight fragments) and the
// LDS-streaming kernels are left to the allocator.
#define UQ_GEMV_OCC __attribute__((amdgpu_waves_per_eu(!XREG || NW < 8 ? 1 : NW / 4)))

// Rows of up to kMaxSegs weight tensors that share x (and dtype, K), laid
// end to end: global row R belongs to segment s with start[s] <= R <
// start[s+1]; its bytes are at w[s] (w2[s] for the gate/up pair) and its
// result goes to y[s]. A single GEMV is one segment.
constexpr int kMaxSegs = 8;
struct Segs {
    int n;
    int start[kMaxSegs + 1];
    const uint8_t *w[kMaxSegs];
    const uint8_t *w2[kMaxSegs];
    float *y[kMaxSegs];
    // one-segment q8k launches: also ysum[r] = add[r] + y[r] (one f32 add,
    // the layer's residual sum) when ysum is set
    const float *add;
    float *ysum;
};
__device__ __forceinline__ int seg_of(const Segs &S, int R) {
    int s = 0;
    for (int i = 1; i < kMaxSegs; i++) s += (i < S.n && R >= S.start[i]) ? 1 : 0;
    return s;
}
// Output address of global row R; R must be wave-uniform, so the segment
// table is read with scalar loads (a per-lane index into the kernel
// arguments would become vector loads and a full vmcnt drain).
template <bool MULTI>
__device__ __forceinline__ float *y_of(const Segs &S, int R) {
    const int sg = MULTI ? __builtin_amdgcn_readfirstlane(seg_of(S, R)) : 0;
    return S.y[sg] + (R - S.start[sg]);
}
// The store of a 4-row batch: lane 16r writes row r's value v; the four
// row addresses are formed wave-uniformly first.
template <bool MULTI>
__device__ __forceinline__ void store4(const Segs &S, int lane, int R0, int nwave, int nvalid, float v) {
    float *p[4];
#pragma unroll
    for (int r = 0; r < 4; r++) p[r] = r < nvalid ? y_of<MULTI>(S, R0 + r * nwave) : nullptr;
    const int r = lane >> 4;
    float *q = r == 0 ? p[0] : r == 1 ? p[1] : r == 2 ? p[2] : p[3];
    if ((lane & 15) == 0 && r < nvalid) *q = v;
}

// One unit = one task of one row. A wave owns rows wave, wave + nwave, ...
// and walks their units in order (the tasks of a row, then the next row); a
// ring of D units keeps that many weight loads in flight, each slot reloaded
// right after it is consumed, and the first D units are issued before the
// activation prep so their HBM latency overlaps it. Rows are taken four at a
// time: a lane accumulates its four partial sums, then one transposed
// reduction (reduce4_rows) yields all four row sums.
// XREG (one task per lane, K <= 4096) keeps the lane's activation digits in
// VGPRs; otherwise they are read from LDS for every unit (then D == 1).
// PAIR: W and W2 (gate, up) share x; writes swiglu(W x, W2 x).
template <class F, bool PAIR, bool XREG, int D, int NW, bool MULTI>
__global__ __launch_bounds__(64 * NW) UQ_GEMV_OCC void gemv_kernel(const Segs S, size_t row_bytes, int K,
                                                               const float *__restrict__ x) {
    static_assert(D == 1 || D == 2 || D == 4, "ring depth divides the 4-row batch");
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int ntask = F::ntasks(K);
    const int T = XREG ? 1 : (ntask + 63) >> 6;  // tasks per lane per row
    const typename F::LC c = F::lane_consts(lane);
    const int wave = blockIdx.x * NW + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
    const int nwave = gridDim.x * NW;
    const int N = S.start[S.n];
    const int nrows = wave < N ? (N - 1 - wave) / nwave + 1 : 0;
    const int U = nrows * T;  // units of this wave

    const float4 x_first = prep_x_first(x, K);
    typename F::Frag f[D], f2[D];
    // single tensor: row pointers advance by a fixed stride; several: each
    // row's segment is looked up (wave-uniform, scalar)
    const size_t stride = (size_t)nwave * row_bytes;
    const uint8_t *pw = S.w[0] + (size_t)wave * row_bytes;
    const uint8_t *pw2 = PAIR ? S.w2[0] + (size_t)wave * row_bytes : nullptr;
    int pr = 0, pt = 0, issued = 0;  // next unit to load: row index, task iteration
    auto issue = [&](typename F::Frag &dst, typename F::Frag &dst2) {
        const int t = lane + 64 * pt;
        if (MULTI) {
            const int R = wave + pr * nwave, sg = __builtin_amdgcn_readfirstlane(seg_of(S, R));
            const size_t off = (size_t)(R - S.start[sg]) * row_bytes;
            pw = S.w[sg] + off;
            if (PAIR) pw2 = S.w2[sg] + off;
        }
        if (t < ntask) {
            dst = F::load_w(pw, t, c);
            if (PAIR) dst2 = F::load_w(pw2, t, c);
        }
        if (++pt == T) {
            pt = 0;
            ++pr;
            if (!MULTI) {
                pw += stride;
                if (PAIR) pw2 += stride;
            }
        }
        ++issued;
    };
#pragma unroll
    for (int d = 0; d < D; d++)
        if (d < U) issue(f[d], f2[d]);

    const XLayout L = x_layout_at<F>(lds, K);
    prep_x<F, 64 * NW>(x, K, L, x_first);
    __syncthreads();
    if (U == 0) return;
    const XView PV{L.xq, L.aux, L.scale, L.gsum, L.NT};
    typename F::XS xr;
    if (XREG && lane < ntask) F::load_x(xr, PV, lane, c);

    for (int rb = 0; rb < nrows; rb += 4) {
        double g[4], u[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            g[r] = 0.0;
            u[r] = 0.0;
            if (rb + r >= nrows) continue;  // wave-uniform
            if (XREG) {
                // one unit per row; its slot is the row's place in the ring
                typename F::Frag &cur = f[r % D], &cur2 = f2[r % D];
                if (lane < ntask) {
                    g[r] = F::dot(cur, xr, c);
                    if (PAIR) u[r] = F::dot(cur2, xr, c);
                }
                if (issued < U) issue(cur, cur2);
            } else {
                for (int tt = 0; tt < T; tt++) {
                    const int t = lane + 64 * tt;
                    if (t < ntask) {
                        typename F::XS xs;
                        F::load_x(xs, PV, t, c);
                        g[r] += F::dot(f[0], xs, c);
                        if (PAIR) u[r] += F::dot(f2[0], xs, c);
                    }
                    if (issued < U) issue(f[0], f2[0]);
                }
            }
        }
        const double G = reduce4_rows(g);
        double Uu = 0.0;
        if (PAIR) Uu = reduce4_rows(u);
        store4<MULTI>(S, lane, wave + rb * nwave, nwave, nrows - rb,
                      PAIR ? swiglu1((float)G, (float)Uu) : (float)G);
    }
}

// Streaming variant of the x-in-VGPR kernel for single tensors (K <= 4096):
// a row is fetched with fully coalesced direct-to-LDS loads
// (global_load_lds_dwordx4: lane i of an instruction writes 16 bytes at
// slot + 16i) into a per-wave ring of S row slots, and each lane then reads
// its task's fragment from the slot. Blocks are laid out at a 16-byte
// aligned pitch (Stage::BP; Q6_K's 210-byte blocks get 224), so chunk k of a
// row is global bytes [blk*210 + 16j, +16) for k = 14*blk + j, and every LDS
// read is aligned. The in-flight row bytes live in LDS, not in VGPRs.
// Synchronisation is per wave: before reading row i the wave waits (vmcnt)
// until at most the ops issued after row i's loads are outstanding: the
// loads of the S-1 later rows (NI instructions each) and the y stores made
// in between; at the tail, where fewer rows follow, it waits for all.
template <class F> struct Stage;
// RP: LDS bytes of one row of up to 16 blocks (a ring slot of the K <= 4096
// streaming kernel); a row's 1 KB loads land at 1024 m within it.
template <> struct Stage<Q6K> {
    static constexpr int BC = 14, BP = 224, BB = kBQ6K;  // chunks per block, LDS pitch, block bytes
    static constexpr int RP = 16 * BP;
    __device__ static Q6KFrag frag(const uint8_t *blk, const Q6K::LC &c) {
        Q6KFrag f;
        f.a = *(const u4 *)(blk + 64 * c.h + 16 * c.u);
        f.b = *(const u4 *)(blk + 64 * c.h + 32 + 16 * c.u);
        f.c = *(const u4 *)(blk + 128 + 32 * c.h + 16 * c.u);
        // scale bytes 8h+u, +2 (s0) and +4, +6 (s1) in bytes 0 and 2, as q6k_load
        f.s0 = *(const uint32_t *)(blk + 192 + 8 * c.h) >> (8 * c.u);
        f.s1 = *(const uint32_t *)(blk + 196 + 8 * c.h) >> (8 * c.u);
        f.dw = *(const uint32_t *)(blk + 208);
        return f;
    }
};
template <> struct Stage<Q4K> {
    static constexpr int BC = 9, BP = 144, BB = kBQ4K;
    static constexpr int RP = 16 * BP;
    __device__ static Q4K::Frag frag(const uint8_t *blk, const Q4K::LC &c) {
        Q4K::Frag f;
        f.h = *(const u4 *)blk;
        f.qa = *(const u4 *)(blk + 16 + 32 * c.p);
        f.qb = *(const u4 *)(blk + 32 + 32 * c.p);
        return f;
    }
};

// 16 bytes per lane from global g into LDS at dst + 16 * lane (dst
// wave-uniform).
// The loads carry the nontemporal hint (cache policy NT = 2): every weight
// byte is read once, and these full-line coalesced loads then stream at a
// markedly higher rate (measured: Q6_K head 101 -> 89 us).
constexpr int UQ_STREAM_CPOL = 2;
__device__ __forceinline__ void lds_dma16(const uint8_t *g, uint8_t *dst) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)dst, 16, 0, UQ_STREAM_CPOL);
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N <= 63, "vmcnt immediate");
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wave priority for long row loops (PRIO): a SIMD's issue arbiter favours
// its oldest wave, and on the 152064-row head (three waves per SIMD, ~50
// rows each) the first wave of each SIMD finished at 77 us, the third at
// 85 us. A PRIO wave sets its priority to (age + row) mod (waves per SIMD)
// for each row, so every wave holds the top priority for an equal share of
// rows. Only launches with many rows per wave use it: the short launches
// keep the plain instantiation.
__device__ __forceinline__ void set_prio(int p) {  // p wave-uniform
    if (p <= 0)
        __builtin_amdgcn_s_setprio(0);
    else if (p == 1)
        __builtin_amdgcn_s_setprio(1);
    else if (p == 2)
        __builtin_amdgcn_s_setprio(2);
    else
        __builtin_amdgcn_s_setprio(3);
}

// PAIR: each row unit is a gate row and an up row (2*NI loads, two slots'
// worth of LDS); MULTI: the row's tensor is looked up in the segment table.
template <class F, int NI, int NW, int S, bool PAIR, bool MULTI, bool PRIO = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW / 4 > 0 ? NW / 4 : 1))) void
gemv_stream_kernel(const Segs Sg, size_t row_bytes, int K, const float *__restrict__ x) {
    static_assert(S == 1 || S == 2 || S == 4, "ring depth divides the 4-row batch");
    using St = Stage<F>;
    constexpr int NT = PAIR ? 2 : 1;   // tensors per row unit
    constexpr int UNIT = NT * NI;      // loads (and KB of LDS) per row unit
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wave = blockIdx.x * NW + wv, nwave = gridDim.x * NW;
    const int ntask = F::ntasks(K);
    const int nchunk = (K >> 8) * St::BC;
    const typename F::LC c = F::lane_consts(lane);
    const int N = Sg.start[Sg.n];
    const int nrows = wave < N ? (N - 1 - wave) / nwave + 1 : 0;
    constexpr int UP = NT * St::RP;    // LDS bytes per row unit
    uint8_t *ring = lds + ((x_lds_bytes<F>(K) + 15) & ~(size_t)15) + (size_t)wv * S * UP;

    uint32_t goff[NI];
    bool gval[NI];
#pragma unroll
    for (int m = 0; m < NI; m++) {
        const int k = lane + 64 * m, b = k / St::BC;
        gval[m] = k < nchunk;
        goff[m] = (uint32_t)(b * St::BB + 16 * (k - b * St::BC));
    }
    auto issue = [&](int i, int slot) {
        if (i < nrows) {  // wave-uniform
            const int R = wave + i * nwave, sg = MULTI ? __builtin_amdgcn_readfirstlane(seg_of(Sg, R)) : 0;
            const size_t off = (size_t)(R - Sg.start[sg]) * row_bytes;
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const uint8_t *row = (t == 0 ? Sg.w[sg] : Sg.w2[sg]) + off;
#pragma unroll
                for (int m = 0; m < NI; m++)
                    if (gval[m]) lds_dma16(row + goff[m], ring + slot * UP + t * St::RP + m * 1024);
            }
        }
    };

    const float4 x_first = prep_x_first(x, K);
#pragma unroll
    for (int sl = 0; sl < S; sl++) issue(sl, sl);
    const XLayout L = x_layout_at<F>(lds, K);
    prep_x<F, 64 * NW>(x, K, L, x_first);
    __syncthreads();
    if (nrows == 0) return;
    const XView PV{L.xq, L.aux, L.scale, L.gsum, L.NT};
    typename F::XS xr;
    if (lane < ntask) F::load_x(xr, PV, lane, c);
    const uint8_t *myblk = ring + (lane >> 2) * St::BP;

    for (int rb = 0; rb < nrows; rb += 4) {
        double g[4], u[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            g[r] = 0.0;
            u[r] = 0.0;
            const int i = rb + r;
            if (i >= nrows) continue;  // wave-uniform
            if constexpr (PRIO) set_prio(((int)wv / 4 + i) % (NW / 4));
            // ops issued after row i's loads: the later rows' loads, and the
            // one y store of the batch that ended among steps i-S .. i-1
            const bool store_between = i >= S && (S == 4 || (S == 2 ? r <= 1 : r == 0));
            if (i + S - 1 < nrows) {
                if (store_between)
                    wait_vm<(S - 1) * UNIT + 1>();
                else
                    wait_vm<(S - 1) * UNIT>();
            } else {
                wait_vm<0>();
            }
            // read only by lanes with a task: no zero fill (it cost a move per dword per row)
            typename F::Frag f, f2;
            const uint8_t *b0 = myblk + (r % S) * UP;
            if (lane < ntask) {
                f = St::frag(b0, c);
                if (PAIR) f2 = St::frag(b0 + St::RP, c);
            }
            // the slot's LDS reads have returned before its next loads land in it
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue(i + S, r % S);
            if (lane < ntask) {
                g[r] = F::dot(f, xr, c);
                if (PAIR) u[r] = F::dot(f2, xr, c);
            }
        }
        const double G = reduce4_rows(g);
        double Uu = 0.0;
        if (PAIR) Uu = reduce4_rows(u);
        store4<MULTI>(Sg, lane, wave + rb * nwave, nwave, nrows - rb,
                      PAIR ? swiglu1((float)G, (float)Uu) : (float)G);
    }
}

// K > 4096 (several tasks per lane and row): rows are still taken four at a
// time, and the loop runs task-outer, row-inner: a lane reads its task's
// activation digits from LDS once and applies them to the four rows, whose
// weight fragments for that task are one load unit. Units run batch-major,
// task-minor; a ring of KT_DEPTH units is in flight, each slot reloaded as
// soon as it is consumed, and the first KT_DEPTH units are issued before the
// prep. Summation per lane is over tasks in order, then reduce4_rows, as in
// gemv_kernel.
constexpr int UQ_KT_NW = 8;
constexpr int UQ_KT_DEPTH = 1;
constexpr int UQ_KT_WPE = 2;
constexpr int KT_NW = UQ_KT_NW;        // waves per workgroup, one workgroup per CU
constexpr int KT_DEPTH = UQ_KT_DEPTH;  // units in flight per wave
template <class F, bool MULTI>
__global__ __launch_bounds__(64 * KT_NW) __attribute__((amdgpu_waves_per_eu(UQ_KT_WPE))) void gemv_kt_kernel(
    const Segs S, size_t row_bytes, int K, const float *__restrict__ x) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int ntask = F::ntasks(K);
    const int T = (ntask + 63) >> 6;
    const typename F::LC c = F::lane_consts(lane);
    const int wave = blockIdx.x * KT_NW + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int nwave = gridDim.x * KT_NW;
    const int N = S.start[S.n];
    const int nrows = wave < N ? (N - 1 - wave) / nwave + 1 : 0;
    const int nb = (nrows + 3) >> 2;
    const int U = nb * T;

    const float4 x_first = prep_x_first(x, K);
    typename F::Frag f[KT_DEPTH][4];
    int iu = 0;  // next unit to load
    auto issue = [&](typename F::Frag(&dst)[4]) {
        const int b = iu / T, t = lane + 64 * (iu - b * T);
        for (int r = 0; r < 4; r++) {
            const int i = 4 * b + r;
            if (i < nrows && t < ntask) {
                const int R = wave + i * nwave, sg = MULTI ? __builtin_amdgcn_readfirstlane(seg_of(S, R)) : 0;
                dst[r] = F::load_w(S.w[sg] + (size_t)(R - S.start[sg]) * row_bytes, t, c);
            }
        }
        ++iu;
    };
#pragma unroll
    for (int d = 0; d < KT_DEPTH; d++)
        if (iu < U) issue(f[d]);

    const XLayout L = x_layout_at<F>(lds, K);
    prep_x<F, 64 * KT_NW, 8>(x, K, L, x_first);
    __syncthreads();
    if (U == 0) return;
    const XView PV{L.xq, L.aux, L.scale, L.gsum, L.NT};

    double g[4] = {0.0, 0.0, 0.0, 0.0};
    for (int u0 = 0; u0 < U; u0 += KT_DEPTH) {
#pragma unroll
        for (int d = 0; d < KT_DEPTH; d++) {
            const int u = u0 + d;
            if (u >= U) break;  // wave-uniform
            const int b = u / T, tt = u - b * T, t = lane + 64 * tt;
            if (t < ntask) {
                typename F::XS xs;
                F::load_x(xs, PV, t, c);
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (4 * b + r < nrows) g[r] += F::dot(f[d][r], xs, c);  // wave-uniform row test
            }
            if (iu < U) issue(f[d]);
            if (tt == T - 1) {
                const double G = reduce4_rows(g);
                store4<MULTI>(S, lane, wave + 4 * b * nwave, nwave, nrows - 4 * b, (float)G);
                for (int q = 0; q < 4; q++) g[q] = 0.0;
            }
        }
    }
}

// 4096 < K <= 16384 (KS = 2..4 slices of 64 tasks): K is split across the
// waves of a workgroup. Wave w owns slice s = w % KS (tasks 64s + lane) and
// row group gi = w / KS; the KS waves of a group walk the same rows (four at
// a time, like gemv_kernel), each keeping its slice's activation digits in
// VGPRs, so every wave has one load unit per row and up to KS_D rows in
// flight. The slice sums of a 4-row batch (reduce4_rows) meet in LDS and
// the slice-0 wave adds them in slice order:
//     y = ((p_0 + p_1) + p_2) + p_3,  p_s = reduce4_rows over slice s.
// Every wave of the workgroup runs the same number of batches (those of its
// first group, which has the most rows), so the per-batch barrier is uniform.
constexpr int UQ_KS_D = 4;  // rows in flight per wave (Q4_K, Q8_0)
constexpr int UQ_KS_D6 = 2;  // Q6_K (larger fragments; 4 would spill at 3 waves per SIMD)

template <class F, int KS, bool MULTI>
__global__ __launch_bounds__(64 * KS_NW) __attribute__((amdgpu_waves_per_eu(3))) void gemv_ks_kernel(
    const Segs S, size_t row_bytes, int K, const float *__restrict__ x) {
    static_assert(KS >= 2 && KS <= 4 && KS_NW % KS == 0, "slices per workgroup");
    constexpr int KS_D = F::kAux ? UQ_KS_D6 : UQ_KS_D;  // kAux: Q6_K
    static_assert(KS_D == 1 || KS_D == 2 || KS_D == 4, "ring depth divides the 4-row batch");
    constexpr int NG = KS_NW / KS;  // row groups per workgroup
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sl = wv % KS, gi = wv / KS;
    const int ntask = F::ntasks(K);
    const int t = 64 * sl + lane;
    const bool act = t < ntask;
    const typename F::LC c = F::lane_consts(lane);
    const int G = blockIdx.x * NG + gi, nG = gridDim.x * NG;  // row group: rows G, G + nG, ...
    const int N = S.start[S.n];
    const int nrows = G < N ? (N - 1 - G) / nG + 1 : 0;
    const int G0 = blockIdx.x * NG;
    const int nb = G0 < N ? ((N - 1 - G0) / nG + 1 + 3) >> 2 : 0;  // batches of the workgroup's first group

    const float4 x_first = prep_x_first(x, K);
    typename F::Frag f[KS_D];
    int pr = 0;  // next row index to load
    auto issue = [&](typename F::Frag &dst) {
        if (pr < nrows && act) {
            const int R = G + pr * nG, sg = MULTI ? __builtin_amdgcn_readfirstlane(seg_of(S, R)) : 0;
            dst = F::load_w(S.w[sg] + (size_t)(R - S.start[sg]) * row_bytes, t, c);
        }
        ++pr;
    };
#pragma unroll
    for (int d = 0; d < KS_D; d++) issue(f[d]);

    const XLayout L = x_layout_at<F>(lds, K);
    double *part = (double *)(lds + ks_part_offset<F>(K));  // [2][NG][KS][4]
    prep_x<F, 64 * KS_NW>(x, K, L, x_first);
    __syncthreads();
    const XView PV{L.xq, L.aux, L.scale, L.gsum, L.NT};
    typename F::XS xr;
    if (act) F::load_x(xr, PV, t, c);

    for (int b = 0; b < nb; b++) {
        double g[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            g[r] = 0.0;
            typename F::Frag &cur = f[r % KS_D];
            if (4 * b + r < nrows && act) g[r] = F::dot(cur, xr, c);  // row test is wave-uniform
            issue(cur);
        }
        const double P = reduce4_rows(g);
        double *pb = part + (size_t)(b & 1) * NG * KS * 4;
        if ((lane & 15) == 0) pb[(gi * KS + sl) * 4 + (lane >> 4)] = P;
        __syncthreads();
        if (sl == 0) {
            double v = 0.0;
            if (lane < 4) {
                v = pb[(gi * KS) * 4 + lane];
                for (int q = 1; q < KS; q++) v += pb[(gi * KS + q) * 4 + lane];
            }
            // lane 16r stores row r: move lane r's sum there
            v = __hiloint2double(__builtin_amdgcn_ds_bpermute(4 * (lane >> 4), __double2hiint(v)),
                                 __builtin_amdgcn_ds_bpermute(4 * (lane >> 4), __double2loint(v)));
            store4<MULTI>(S, lane, G + 4 * b * nG, nG, nrows - 4 * b, (float)v);
        }
    }
}

// gemv_ks_kernel's split with the weights streamed into LDS (Q4_K / Q6_K,
// 4096 < K <= 20480, sks_slices): wave w owns slice s = w % KS (blocks
// [16 s, 16 s + 16))
// of row group gi = w / KS. Each wave moves its slice of a row into its own
// ring slot with coalesced direct-to-LDS nontemporal loads (NI per row, D
// rows in flight), as gemv_stream_kernel does for whole rows, and reads its
// lane's task from there. Slice sums of a 4-row batch meet in LDS and the
// slice-0 wave adds them in slice order, as in gemv_ks_kernel.
template <class F, int NI, int KS, int NG, int D, bool MULTI>
__global__ __launch_bounds__(64 * KS * NG) void gemv_stream_ks_kernel(const Segs Sg, size_t row_bytes, int K,
                                                                     const float *__restrict__ x) {
    static_assert(D == 1 || D == 2 || D == 4, "ring depth divides the 4-row batch");
    using St = Stage<F>;
    constexpr int NW = KS * NG;
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sl = wv % KS, gi = wv / KS;
    const int ntask = F::ntasks(K);
    const int t = 64 * sl + lane;
    const bool act = t < ntask;
    const typename F::LC c = F::lane_consts(lane);
    const int G = blockIdx.x * NG + gi, nG = gridDim.x * NG;  // row group: rows G, G + nG, ...
    const int N = Sg.start[Sg.n];
    const int nrows = G < N ? (N - 1 - G) / nG + 1 : 0;
    const int G0 = blockIdx.x * NG;
    const int nb = G0 < N ? ((N - 1 - G0) / nG + 1 + 3) >> 2 : 0;  // batches of the workgroup's first group
    const int nblk = K >> 8;
    const int nch = (min(nblk, 16 * sl + 16) - 16 * sl) * St::BC;  // 16-byte chunks of this slice
    // every one of the NI loads of a row has an active lane, so each is issued
    // and counted; a short last slice instead waits for all its loads
    const bool full = nch > 64 * (NI - 1);
    const size_t part_off = (x_lds_bytes<F>(K) + 15) & ~(size_t)15;
    double *part = (double *)(lds + part_off);  // [2][NG][KS][4]
    uint8_t *ring = lds + part_off + (size_t)2 * NG * KS * 4 * 8 + (size_t)wv * D * NI * 1024;

    uint32_t goff[NI];
    bool gval[NI];
#pragma unroll
    for (int m = 0; m < NI; m++) {
        const int k = lane + 64 * m, b = k / St::BC;
        gval[m] = k < nch;
        goff[m] = (uint32_t)((16 * sl + b) * St::BB + 16 * (k - b * St::BC));
    }
    auto issue = [&](int i, int slot) {
        if (i < nrows) {  // wave-uniform
            const int R = G + i * nG, sg = MULTI ? __builtin_amdgcn_readfirstlane(seg_of(Sg, R)) : 0;
            const uint8_t *row = Sg.w[sg] + (size_t)(R - Sg.start[sg]) * row_bytes;
#pragma unroll
            for (int m = 0; m < NI; m++)
                if (gval[m]) lds_dma16(row + goff[m], ring + (slot * NI + m) * 1024);
        }
    };

    const float4 x_first = prep_x_first(x, K);
#pragma unroll
    for (int d = 0; d < D; d++) issue(d, d);
    const XLayout L = x_layout_at<F>(lds, K);
    prep_x<F, 64 * NW>(x, K, L, x_first);
    __syncthreads();
    if (nb == 0) return;  // the whole workgroup: no rows
    const XView PV{L.xq, L.aux, L.scale, L.gsum, L.NT};
    typename F::XS xr;
    if (act) F::load_x(xr, PV, t, c);
    const uint8_t *myblk = ring + (lane >> 2) * St::BP;

    for (int b = 0; b < nb; b++) {
        double g[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            g[r] = 0.0;
            const int i = 4 * b + r;
            if (i < nrows) {  // wave-uniform
                // ops issued after row i's loads: the later rows' loads and,
                // for the slice-0 wave, the y store of the previous batch
                const bool store_between = sl == 0 && b > 0 && (D == 4 || (D == 2 ? r <= 1 : r == 0));
                if (full && i + D - 1 < nrows) {
                    if (store_between)
                        wait_vm<(D - 1) * NI + 1>();
                    else
                        wait_vm<(D - 1) * NI>();
                } else {
                    wait_vm<0>();
                }
                typename F::Frag f;
                if (act) f = St::frag(myblk + (r % D) * NI * 1024, c);
                // the slot's LDS reads have returned before its next loads land in it
                __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                issue(i + D, r % D);
                if (act) g[r] = F::dot(f, xr, c);
            }
        }
        const double P = reduce4_rows(g);
        double *pb = part + (size_t)(b & 1) * NG * KS * 4;
        if ((lane & 15) == 0) pb[(gi * KS + sl) * 4 + (lane >> 4)] = P;
        __syncthreads();
        if (sl == 0) {
            double v = 0.0;
            if (lane < 4) {
                v = pb[(gi * KS) * 4 + lane];
                for (int q = 1; q < KS; q++) v += pb[(gi * KS + q) * 4 + lane];
            }
            // lane 16r stores row r: move lane r's sum there
            v = __hiloint2double(__builtin_amdgcn_ds_bpermute(4 * (lane >> 4), __double2hiint(v)),
                                 __builtin_amdgcn_ds_bpermute(4 * (lane >> 4), __double2loint(v)));
            store4<MULTI>(Sg, lane, G + 4 * b * nG, nG, nrows - 4 * b, (float)v);
        }
    }
}

// Generic fallback (F32 rows, Q8_0 with K % 64 != 0, K beyond the LDS
// budget): one wave per row, f32 dequantization (exact: one rounding for
// Q4_K, none for Q6_K/Q8_0/F32, quants.rs:129-131, :170) and f64
// accumulation of the exact products x*w.
__device__ __forceinline__ float deq_elem(uq_dtype dt, const uint8_t *row, int e) {
    if (dt == UQ_F32) return ((const float *)row)[e];
    if (dt == UQ_Q8_0) {
        const uint8_t *b = row + (e >> 5) * BQ8_0;
        return f16_bits_exact(b[0] | (b[1] << 8)) * (float)(int8_t)b[2 + (e & 31)];
    }
    if (dt == UQ_Q4_K) {
        const uint8_t *b = row + (e >> 8) * BQ4K;
        const int l = e & 255, g = l >> 5;
        const uint8_t *s = b + 4;
        uint32_t sc, m;
        if (g < 4) {
            sc = s[g] & 63;
            m = s[g + 4] & 63;
        } else {
            sc = (s[g + 4] & 0xF) | ((s[g - 4] >> 6) << 4);
            m = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
        }
        const uint8_t byte = b[16 + 32 * (g >> 1) + (l & 31)];
        const uint32_t nib = (g & 1) ? (byte >> 4) : (byte & 0xF);
        return (f16_bits_exact(b[0] | (b[1] << 8)) * (float)sc) * (float)nib -
               f16_bits_exact(b[2] | (b[3] << 8)) * (float)m;
    }
    const uint8_t *b = row + (e >> 8) * BQ6K;
    const int l = e & 255;
    const uint8_t byte = b[64 * (l / 128) + (l % 64)];
    const int nib = ((l / 64) % 2 == 0) ? (byte & 0xF) : (byte >> 4);
    const int hi2 = (b[128 + (l % 32) + 32 * (l / 128)] >> (2 * ((l % 128) / 32))) & 3;
    return f16_bits_exact(b[208] | (b[209] << 8)) *
           ((float)(int8_t)b[192 + l / 16] * (float)((nib | (hi2 << 4)) - 32));
}

__global__ __launch_bounds__(TPB) void gemv_generic_kernel(uq_dtype dt, const uint8_t *__restrict__ W,
                                                           const uint8_t *__restrict__ W2,
                                                           size_t row_bytes, int K, int N,
                                                           const float *__restrict__ x,
                                                           float *__restrict__ y) {
    const int lane = threadIdx.x & 63;
    for (int row = blockIdx.x * WAVES + (threadIdx.x >> 6); row < N; row += gridDim.x * WAVES) {
        const uint8_t *R = W + (size_t)row * row_bytes;
        double g = 0.0, u = 0.0;
        for (int e = lane; e < K; e += 64) {
            g = fma((double)x[e], (double)deq_elem(dt, R, e), g);
            if (W2) u = fma((double)x[e], (double)deq_elem(dt, W2 + (size_t)row * row_bytes, e), u);
        }
        g = wave_sum_d(g);
        if (W2) {
            u = wave_sum_d(u);
            if (lane == 0) y[row] = swiglu1((float)g, (float)u);
        } else if (lane == 0) {
            y[row] = (float)g;
        }
    }
}

// Workgroups for a row-walking kernel: exactly the number that are resident
// at once (occupancy from VGPRs/LDS), so no workgroup waits for a second
// round, then trimmed so every wave walks the same number of rows.
int blocks_per_cu(const void *kernel, size_t lds, int tpb) {
    static std::mutex mu;
    static std::map<std::pair<const void *, size_t>, int> cache;
    std::lock_guard<std::mutex> g(mu);
    auto it = cache.find({kernel, lds});
    if (it != cache.end()) return it->second;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, tpb, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    cache[{kernel, lds}] = per_cu;
    return per_cu;
}

int resident_grid(const void *kernel, size_t lds, int N, int nw = WAVES) {
    int per_cu = blocks_per_cu(kernel, lds, 64 * nw);
    const int max_waves = num_cus() * per_cu * nw;
    const int rows_per_wave = (N + max_waves - 1) / max_waves;
    const int waves = (N + rows_per_wave - 1) / rows_per_wave;
    return (waves + nw - 1) / nw;
}

// Launch shape of the x-in-VGPR kernels, per format: one workgroup per CU
// (NW waves) so the activation prep runs once per CU, with D units in flight
// per wave. Q6_K: 12 waves (3 per SIMD, <= 168 VGPRs) with two units in
// flight; Q4_K and Q8_0: 16 waves (4 per SIMD, <= 128 VGPRs), one unit; the
// gate/up pair: 12 waves, one unit (two fragments).
constexpr int UQ_Q4K_NW = 16;
constexpr int UQ_Q4K_D = 1;
constexpr int UQ_PAIR_NW = 12;
constexpr int UQ_PAIR_D = 1;
template <class F> struct Shape { static constexpr int NW = UQ_Q4K_NW, D = UQ_Q4K_D; };
constexpr int UQ_Q6K_NW = 12;
constexpr int UQ_Q6K_D = 2;
template <> struct Shape<Q6K> { static constexpr int NW = UQ_Q6K_NW, D = UQ_Q6K_D; };

// Launch shape of the streaming kernel (one workgroup per CU, SNW waves,
// SS rows per wave in flight), measured on the 152064 x 4096 Q6_K head and
// the 4096 / 12288 x 4096 Q4_K projections.
constexpr int UQ_STREAM_Q6K_NW = 12;
constexpr int UQ_STREAM_Q6K_S = 1;
constexpr int UQ_STREAM_Q4K_NW = 16;
constexpr int UQ_STREAM_Q4K_S = 1;
constexpr int UQ_STREAM_PAIR_NW = 12;
constexpr int UQ_STREAM_PAIR_S = 1;
constexpr int UQ_STREAM_ON = 1;
template <class F> struct StreamShape { static constexpr int NW = UQ_STREAM_Q4K_NW, S = UQ_STREAM_Q4K_S; };
template <> struct StreamShape<Q6K> { static constexpr int NW = UQ_STREAM_Q6K_NW, S = UQ_STREAM_Q6K_S; };

constexpr int kPrioRows = 16;  // rows per wave from which the PRIO instantiation runs

template <class F, int NI, bool PAIR, bool MULTI>
hipError_t launch_stream(const Segs &S, size_t row_bytes, int K, const float *x, hipStream_t s) {
    constexpr int SNW = PAIR ? UQ_STREAM_PAIR_NW : StreamShape<F>::NW, SS = PAIR ? UQ_STREAM_PAIR_S : StreamShape<F>::S;
    const int N = S.start[S.n];
    const size_t l = ((x_lds_bytes<F>(K) + 15) & ~(size_t)15) + (size_t)SNW * SS * (PAIR ? 2 : 1) * Stage<F>::RP;
    const void *k = (const void *)gemv_stream_kernel<F, NI, SNW, SS, PAIR, MULTI>;
    const hipError_t e = allow_lds(k, l);
    if (e != hipSuccess) return e;
    const int grid = resident_grid(k, l, N, SNW);
    if constexpr (!PAIR && !MULTI) {
        if ((N + grid * SNW - 1) / (grid * SNW) >= kPrioRows) {  // rows per wave
            const void *kp = (const void *)gemv_stream_kernel<F, NI, SNW, SS, false, false, true>;
            const hipError_t ep = allow_lds(kp, l);
            if (ep != hipSuccess) return ep;
            hipLaunchKernelGGL((gemv_stream_kernel<F, NI, SNW, SS, false, false, true>), dim3(grid), dim3(64 * SNW),
                               l, s, S, row_bytes, K, x);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((gemv_stream_kernel<F, NI, SNW, SS, PAIR, MULTI>), dim3(grid), dim3(64 * SNW), l, s, S,
                       row_bytes, K, x);
    return hipGetLastError();
}

constexpr int UQ_STREAM_KS = 1;
// gemv_stream_ks_kernel for the rows that sks_slices splits (K <= 20480):
// 2-3 slices run 4 row groups with 2 rows in flight, 4-5 slices 3 groups
// with 1 (sks_shape; the template arguments below follow it). *done
// reports whether it was launched.
template <class F, bool MULTI>
hipError_t launch_stream_ks(const Segs &S, size_t row_bytes, int K, const float *x, hipStream_t s, bool *done) {
    constexpr int NI = (16 * Stage<F>::BC + 63) / 64;
    static_assert(NI == F::kSksLoads, "1 KB loads per row slice");
    const int ks = sks_slices<F>(K);
    *done = false;
    if (!ks) return hipSuccess;
    int ng, d;
    sks_shape(ks, ng, d);
    const size_t l = sks_lds<F>(K, ks);
    auto go = [&](auto kern) -> hipError_t {
        const void *k = (const void *)kern;
        hipError_t e = allow_lds(k, l);
        if (e != hipSuccess) return e;
        const int N = S.start[S.n];
        // one workgroup per CU, ng row groups each, rows dealt round-robin to the groups
        const int rpg = (N + num_cus() * ng - 1) / (num_cus() * ng);
        const int grid = (N + rpg * ng - 1) / (rpg * ng);
        hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * ks * ng), l, s, S, row_bytes, K, x);
        *done = true;
        return hipGetLastError();
    };
    if (ks == 2) return go(gemv_stream_ks_kernel<F, NI, 2, 4, 2, MULTI>);
    if (ks == 3) return go(gemv_stream_ks_kernel<F, NI, 3, 4, 2, MULTI>);
    if (ks == 4) return go(gemv_stream_ks_kernel<F, NI, 4, 3, 1, MULTI>);
    return go(gemv_stream_ks_kernel<F, NI, 5, 3, 1, MULTI>);
}

template <class F, bool PAIR, bool MULTI>
hipError_t launch_fast_m(const Segs &S, size_t row_bytes, int K, const float *x, hipStream_t s) {
    const int N = S.start[S.n];
    const size_t lds = x_lds_bytes<F>(K);
    // Q4_K / Q6_K rows with K <= 4096 stream through LDS
    if constexpr (std::is_same<F, Q6K>::value || std::is_same<F, Q4K>::value) {
        if (F::ntasks(K) <= 64 && UQ_STREAM_ON) {
            const int ni = ((K >> 8) * Stage<F>::BC + 63) / 64;
            if (ni == 4) return launch_stream<F, 4, PAIR, MULTI>(S, row_bytes, K, x, s);
            if (ni == 3) return launch_stream<F, 3, PAIR, MULTI>(S, row_bytes, K, x, s);
            if (ni == 2) return launch_stream<F, 2, PAIR, MULTI>(S, row_bytes, K, x, s);
            return launch_stream<F, 1, PAIR, MULTI>(S, row_bytes, K, x, s);
        }
    }
    if (F::ntasks(K) <= 64) {
        constexpr int NW = PAIR ? UQ_PAIR_NW : Shape<F>::NW, D = PAIR ? UQ_PAIR_D : Shape<F>::D;
        const void *k = (const void *)gemv_kernel<F, PAIR, true, D, NW, MULTI>;
        hipLaunchKernelGGL((gemv_kernel<F, PAIR, true, D, NW, MULTI>), dim3(resident_grid(k, lds, N, NW)),
                           dim3(64 * NW), lds, s, S, row_bytes, K, x);
    } else if constexpr (!PAIR) {
        if constexpr (std::is_same<F, Q6K>::value || std::is_same<F, Q4K>::value) {
            if (UQ_STREAM_KS && sks_slices<F>(K)) {
                bool done = false;
                const hipError_t e = launch_stream_ks<F, MULTI>(S, row_bytes, K, x, s, &done);
                if (e != hipSuccess || done) return e;
            }
        }
        const int ks = kslices<F>(K);
        const size_t lds_ks = ks_lds_bytes<F>(K);
        if (ks) {
            auto go = [&](auto kern, int nslice) {
                // one workgroup per CU (as resident), KS_NW / nslice row groups each
                const int ng = KS_NW / nslice;
                const int max_groups = num_cus() * blocks_per_cu((const void *)kern, lds_ks, 64 * KS_NW) * ng;
                const int rows_per_group = (N + max_groups - 1) / max_groups;
                const int groups = (N + rows_per_group - 1) / rows_per_group;
                hipLaunchKernelGGL(kern, dim3((groups + ng - 1) / ng), dim3(64 * KS_NW), lds_ks, s, S, row_bytes, K,
                                   x);
            };
            if (ks == 2)
                go(gemv_ks_kernel<F, 2, MULTI>, 2);
            else if (ks == 3)
                go(gemv_ks_kernel<F, 3, MULTI>, 3);
            else
                go(gemv_ks_kernel<F, 4, MULTI>, 4);
        } else {
            const void *k = (const void *)gemv_kt_kernel<F, MULTI>;
            hipLaunchKernelGGL((gemv_kt_kernel<F, MULTI>), dim3(resident_grid(k, lds, N, KT_NW)), dim3(64 * KT_NW),
                               lds, s, S, row_bytes, K, x);
        }
    } else {
        const void *k = (const void *)gemv_kernel<F, PAIR, false, 1, WAVES, MULTI>;
        hipLaunchKernelGGL((gemv_kernel<F, PAIR, false, 1, WAVES, MULTI>), dim3(resident_grid(k, lds, N)), dim3(TPB),
                           lds, s, S, row_bytes, K, x);
    }
    return hipGetLastError();
}
template <class F, bool PAIR>
hipError_t launch_fast(const Segs &S, size_t row_bytes, int K, const float *x, hipStream_t s) {
    if (PAIR || S.n == 1) return launch_fast_m<F, PAIR, false>(S, row_bytes, K, x, s);
    return launch_fast_m<F, false, true>(S, row_bytes, K, x, s);
}

// All segments share dtype, K and row_bytes; pair = S.w2 holds the up rows.
hipError_t launch_segs(uq_dtype dt, int K, size_t row_bytes, const Segs &S, bool pair, const float *x,
                       hipStream_t s) {
    if (S.start[S.n] == 0) return hipSuccess;
    // Q4_K / Q6_K rows beyond the 64 KB layout budget still take the fast
    // path when the streaming split holds them (K <= 20480)
    if (dt == UQ_Q4_K && (x_lds_bytes<Q4K>(K) <= kLdsCap || (!pair && UQ_STREAM_KS && sks_slices<Q4K>(K))))
        return pair ? launch_fast<Q4K, true>(S, row_bytes, K, x, s) : launch_fast<Q4K, false>(S, row_bytes, K, x, s);
    if (dt == UQ_Q6_K && (x_lds_bytes<Q6K>(K) <= kLdsCap || (!pair && UQ_STREAM_KS && sks_slices<Q6K>(K))))
        return pair ? launch_fast<Q6K, true>(S, row_bytes, K, x, s) : launch_fast<Q6K, false>(S, row_bytes, K, x, s);
    if (dt == UQ_Q8_0 && K % 64 == 0 && x_lds_bytes<Q80>(K) <= kLdsCap)
        return pair ? launch_fast<Q80, true>(S, row_bytes, K, x, s) : launch_fast<Q80, false>(S, row_bytes, K, x, s);
    for (int i = 0; i < S.n; i++) {
        const int N = S.start[i + 1] - S.start[i];
        if (N == 0) continue;
        int grid = (N + WAVES - 1) / WAVES;
        if (grid > num_cus() * 8) grid = num_cus() * 8;
        hipLaunchKernelGGL(gemv_generic_kernel, dim3(grid), dim3(TPB), 0, s, dt, S.w[i], pair ? S.w2[i] : nullptr,
                           row_bytes, K, N, x, S.y[i]);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

Segs one_seg(const WeightsView &w, const uint8_t *w2, float *y) {
    Segs S{};
    S.n = 1;
    S.start[0] = 0;
    S.start[1] = w.dim_out;
    S.w[0] = w.bytes;
    S.w2[0] = w2;
    S.y[0] = y;
    return S;
}

// ---------------------------- gemv_quant_q8k -------------------------------
// quantize_q8_k (quants.rs:250-290) of one 256-block by one wave into LDS:
// q = 64 dwords of qs, bs = 16 bsums, *d = block scale.
// v: the lane's four values of the block (elements 4 lane .. 4 lane + 3).
__device__ __forceinline__ void quantize_vals_lds(const float (&v)[4], int lane, uint32_t *q, int *bs, float *dq) {
    float am = 0.0f, mx = 0.0f;
    for (int i = 0; i < 4; i++) {
        const float a = fabsf(v[i]);
        if (a > am) {
            am = a;
            mx = v[i];
        }
    }
    wave_first_absmax(am, mx);  // first strict argmax of |x|
    uint32_t packed = 0;
    int s = 0;
    if (am != 0.0f) {
        const float iscale = __fdiv_rn(-127.0f, mx);
        for (int i = 0; i < 4; i++) {
            const float val = __fadd_rn(__fmul_rn(iscale, v[i]), 12582912.0f);
            int qv = (int)(__float_as_uint(val) & 0x007FFFFFu) - 0x00400000;
            qv = qv < 127 ? qv : 127;
            packed |= ((uint32_t)qv & 0xFF) << (8 * i);
            s += qv;
        }
        if (lane == 0) *dq = __fdiv_rn(1.0f, iscale);
    } else if (lane == 0) {
        *dq = 0.0f;
    }
    q[lane] = packed;
    s = group4_sum_i(s);
    if ((lane & 3) == 0) bs[lane >> 2] = s;
}

// Blocks first, first + step, ... < nblk of x by one wave, as
// quantize_vals_lds; the loads of four blocks issue before any of them is
// processed, so their latencies overlap.
__device__ __forceinline__ void quantize_blocks_lds(const float *__restrict__ x, int first, int step, int nblk,
                                                    int lane, uint32_t *q, int *bs, float *d8) {
    for (int b0 = first; b0 < nblk; b0 += 4 * step) {
        float v[4][4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int b = b0 + j * step;
            if (b < nblk)  // wave-uniform
#pragma unroll
                for (int i = 0; i < 4; i++) v[j][i] = x[256 * b + lane * 4 + i];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int b = b0 + j * step;
            if (b < nblk) quantize_vals_lds(v[j], lane, q + 64 * b, bs + 16 * b, d8 + b);
        }
    }
}

// The q8k input of a launch: x itself, or its row norm (nrm.w set): the
// elements rmsnorm_kernel forms (kernels.rs:61-78), (t * scale) * w with t =
// x (+ xb) and scale = 1 / sqrt(mean + eps), mean the sequential f64 sum of
// t*t over K (the bound-or-replay sum of seq_sum_f32). A wave loads the t
// and w of the blocks it quantizes (b = wv, wv + nw, ..., at most four: K <=
// 4096 with four or more waves) once, before the workgroup's sum; workgroup 0
// also writes the normalised row and x + xb where asked. qtmp is the prep
// area (at least 256 bytes, free until the quantization writes it).
template <int TPB>
__device__ __forceinline__ void q8k_input(const float *__restrict__ x, const RowNorm &nrm, int K, int wv, int nw,
                                          int lane, uint32_t *qtmp, int *bst, float *d8) {
    const int nblk = K >> 8;
    if (!nrm.w) {
        quantize_blocks_lds(x, wv, nw, nblk, lane, qtmp, bst, d8);
        return;
    }
    const float *xb = nrm.xb, *w = nrm.w;
    float t[4][4], wt[4][4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int b = wv + j * nw;
        if (b < nblk)  // wave-uniform
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int e = 256 * b + lane * 4 + i;
                t[j][i] = xb ? __fadd_rn(x[e], xb[e]) : x[e];
                wt[j][i] = w[e];
            }
    }
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < 4; j++)
        if (wv + j * nw < nblk)
#pragma unroll
            for (int i = 0; i < 4; i++) s += (double)__fmul_rn(t[j][i], t[j][i]);
    const double S = block_sum_d<TPB>(s, (double *)qtmp);
    const double dn = (double)K;
    auto val = [&](int e) { return xb ? __fadd_rn(x[e], xb[e]) : x[e]; };
    const float mean = seq_sum_f32<TPB>(val, K, S, [dn](double u) { return (float)(u / dn); }, (float *)qtmp + 64);
    const float scale = __fdiv_rn(1.0f, sqrtf_cr(__fadd_rn(mean, nrm.eps)));
    const bool out = blockIdx.x == 0 && nrm.xn_out;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int b = wv + j * nw;
        if (b < nblk) {
            float y[4];
#pragma unroll
            for (int i = 0; i < 4; i++) y[i] = __fmul_rn(__fmul_rn(t[j][i], scale), wt[j][i]);
            quantize_vals_lds(y, lane, qtmp + 64 * b, bst + 16 * b, d8 + b);
            if (out)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int e = 256 * b + lane * 4 + i;
                    nrm.xn_out[e] = y[i];
                    if (nrm.xsum_out) nrm.xsum_out[e] = t[j][i];
                }
        }
    }
}

struct Q8KLayout {
    size_t xq, d8, region, total;  // byte offsets
    int R;                         // rows per epilogue batch
};

template <class F>
__host__ __device__ inline Q8KLayout q8k_layout(int K) {
    const int nblk = K >> 8, ntask = 4 * nblk;
    const int dw = F::kDw;
    Q8KLayout L;
    L.xq = 0;
    L.d8 = (size_t)ntask * dw * 4;
    L.region = (L.d8 + (size_t)nblk * 4 + 15) & ~(size_t)15;
    int R = (int)(32768 / ((size_t)WAVES * nblk * 40));
    L.R = R < 1 ? 1 : (R > 8 ? 8 : R);
    const size_t prep = (size_t)K + (size_t)(K / 16) * 4;
    const size_t recs = (size_t)WAVES * L.R * nblk * 40;
    L.total = L.region + (prep > recs ? prep : recs);
    return L;
}

template <class F, bool CACHED, bool MULTI>
__global__ __launch_bounds__(TPB) void gemv_q8k_kernel(const Segs S, size_t row_bytes, int K,
                                                       const float *__restrict__ x) {
    extern __shared__ __align__(16) uint8_t lds[];
    const Q8KLayout L = q8k_layout<F>(K);
    const int nblk = K >> 8, ntask = 4 * nblk, R = L.R;
    uint32_t *xq = (uint32_t *)(lds + L.xq);
    float *d8 = (float *)(lds + L.d8);
    uint32_t *qtmp = (uint32_t *)(lds + L.region);
    int *bst = (int *)(lds + L.region + K);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;

    quantize_blocks_lds(x, wid, WAVES, nblk, lane, qtmp, bst, d8);
    __syncthreads();
    for (int t = threadIdx.x; t < ntask; t += TPB)
        F::build_task(xq + (size_t)t * F::kDw, qtmp + 64 * (t >> 2), bst + 16 * (t >> 2), t & 3);
    __syncthreads();  // the prep region becomes the per-wave record area

    uint32_t *rec = (uint32_t *)(lds + L.region) + (size_t)wid * R * nblk * 10;
    const typename F::LC c = F::lane_consts(lane);
    const int wave = blockIdx.x * WAVES + wid, nwave = gridDim.x * WAVES;
    const int iters = (ntask + 63) / 64;
    typename F::XS xs0;
    if (CACHED && lane < ntask) F::load_x(xs0, xq, lane);

    const int N = S.start[S.n];
    int slot = 0;
    for (int row = wave; row < N; row += nwave) {
        const int sg = MULTI ? __builtin_amdgcn_readfirstlane(seg_of(S, row)) : 0;
        const uint8_t *Rw = S.w[sg] + (size_t)(row - S.start[sg]) * row_bytes;
        for (int it = 0; it < iters; it++) {
            const int t = lane + 64 * it;
            int S[8] = {0, 0, 0, 0, 0, 0, 0, 0}, M = 0;
            uint32_t h = 0;
            if (t < ntask) {
                typename F::XS xsl;
                if (!CACHED) F::load_x(xsl, xq, t);
                const typename F::Frag f = F::load_w(Rw, t, c);
                F::dot(f, CACHED ? xs0 : xsl, c, S, M);
                h = F::hdr(f);
            }
            // the four tasks of a block are one lane quad: sum them
#pragma unroll
            for (int k = 0; k < 8; k++) S[k] = group4_sum_i(S[k]);
            if (F::kMin) M = group4_sum_i(M);
            if (t < ntask) {
                const int q = t & 3;
                uint32_t *r = rec + ((size_t)slot * nblk + (t >> 2)) * 10;
                r[2 * q] = (uint32_t)S[2 * q];
                r[2 * q + 1] = (uint32_t)S[2 * q + 1];
                if (q == 0) {
                    r[8] = (uint32_t)M;
                    r[9] = h;
                }
            }
        }
        slot++;
        if (slot == R || row + nwave >= N) {
            // epilogue (quants.rs:343-358 / :402-411): lane (r, k) replays
            // sums[k] += d*sumi[k] over the blocks in order; k = 0 also
            // replays sumf -= dmin*minsum; then s = sumf + sums[0] + ... + sums[7].
            __builtin_amdgcn_wave_barrier();
            q8k_fold<F::kMin>(rec, nblk * 10, d8, slot, 0, nblk, lane);
            __builtin_amdgcn_wave_barrier();
            const int r = lane >> 3, k = lane & 7;
            float sums = 0.0f, sumf = 0.0f;
            if (r < slot) q8k_replay<F::kMin>(rec + (size_t)(r) * nblk * 10, nblk, k, sums, sumf);
            // Q6_K: sumf stays 0.0f, matching `let mut s = 0.0f32`; lane k = 0 holds s
            const float s = group8_chain_first(sumf, sums);
            if (k == 0 && r < slot) {
                const int Rr = row - (slot - 1 - r) * nwave, so = MULTI ? seg_of(S, Rr) : 0;
                S.y[so][Rr - S.start[so]] = s;
                if (!MULTI && S.ysum) S.ysum[Rr] = __fadd_rn(S.add[Rr], s);
            }
            __builtin_amdgcn_wave_barrier();
            slot = 0;
        }
    }
}

// Streaming variant of gemv_q8k_kernel (bit-exact, same arithmetic) for one
// Q4_K / Q6_K tensor or a batch, K <= 12288: rows arrive through the
// per-wave LDS ring of gemv_stream_kernel (coalesced nontemporal
// direct-to-LDS loads, one row in flight per wave, issued before the wave
// computes the previous one), instead of per-lane loads into VGPRs. A lane
// owns T tasks of a row (t = lane + 64 tt); with T = 1 its x record stays in
// VGPRs, otherwise each task's record is read from LDS. The lane-quad sums,
// the per-wave row records and the reference-order epilogue are those of
// gemv_q8k_kernel.
template <class F> struct Q8Base;
template <> struct Q8Base<Q6KQ8> { using T = Q6K; };
template <> struct Q8Base<Q4KQ8> { using T = Q4K; };

constexpr size_t kQ8SLds = 160 * 1024;  // LDS of one workgroup (one per CU)

struct Q8SLayout {
    size_t xq, d8, region, ring, total;  // byte offsets
    int R;                               // rows per epilogue batch (<= 8; 0: does not fit)
};
// NT = 2: gate/up pairs (two rows per ring unit, two record sets per wave)
template <class F>
__host__ __device__ inline Q8SLayout q8k_stream_layout(int K, int nw, int ni, int nt = 1) {
    const int nblk = K >> 8, ntask = 4 * nblk;
    Q8SLayout L;
    L.xq = 0;
    L.d8 = (size_t)ntask * F::kDw * 4;
    L.region = (L.d8 + (size_t)nblk * 4 + 15) & ~(size_t)15;
    const size_t ring = (size_t)nw * nt * ni * 1024, prep = (size_t)K + (size_t)(K / 16) * 4;
    const size_t left = kQ8SLds > L.region + ring ? kQ8SLds - L.region - ring : 0;
    int R = (int)(left / ((size_t)nw * nt * nblk * 40 + 16));
    L.R = R > 8 ? 8 : R;
    const size_t recs = (size_t)nw * nt * (L.R > 0 ? L.R : 1) * nblk * 40;
    L.ring = (L.region + (prep > recs ? prep : recs) + 15) & ~(size_t)15;
    L.total = L.ring + ring;
    return L;
}

// PAIR (T = 1, one segment): a ring unit is gate row r (Sg.w) and up row r
// (Sg.w2); the wave keeps a record set for each and stores g (Sg.y[0]), u
// (Sg.y[1]) and h = swiglu(g, u) (Sg.y[2]).
template <class F, int T, int NW, bool MULTI, bool PAIR = false, bool PRIO = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW / 4 > 0 ? NW / 4 : 1))) void
gemv_q8k_stream_kernel(const Segs Sg, size_t row_bytes, int K, const float *__restrict__ x, const RowNorm nrm) {
    static_assert(!PAIR || (T == 1 && !MULTI), "pairs: one segment, K <= 4096");
    using St = Stage<typename Q8Base<F>::T>;
    constexpr int NI = (16 * T * St::BC + 63) / 64;  // 1 KB loads per row (K <= 4096 T)
    constexpr int NT = PAIR ? 2 : 1;                 // rows per ring unit
    extern __shared__ __align__(16) uint8_t lds[];
    const Q8SLayout L = q8k_stream_layout<F>(K, NW, NI, NT);
    const int nblk = K >> 8, ntask = 4 * nblk, R = L.R;
    uint32_t *xq = (uint32_t *)(lds + L.xq);
    float *d8 = (float *)(lds + L.d8);
    uint32_t *qtmp = (uint32_t *)(lds + L.region);
    int *bst = (int *)(lds + L.region + K);
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wave = blockIdx.x * NW + wv, nwave = gridDim.x * NW;
    const int N = Sg.start[Sg.n];
    const int nrows = wave < N ? (N - 1 - wave) / nwave + 1 : 0;
    const int nchunk = nblk * St::BC;
    uint8_t *ring = lds + L.ring + (size_t)wv * NT * NI * 1024;

    uint32_t goff[NI];
    bool gval[NI];
#pragma unroll
    for (int m = 0; m < NI; m++) {
        const int k = lane + 64 * m, b = k / St::BC;
        gval[m] = k < nchunk;
        goff[m] = (uint32_t)(b * St::BB + 16 * (k - b * St::BC));
    }
    auto issue = [&](int i) {
        if (i < nrows) {  // wave-uniform
            const int Rw = wave + i * nwave, sg = MULTI ? __builtin_amdgcn_readfirstlane(seg_of(Sg, Rw)) : 0;
#pragma unroll
            for (int u = 0; u < NT; u++) {
                const uint8_t *row = (u == 0 ? Sg.w[sg] : Sg.w2[sg]) + (size_t)(Rw - Sg.start[sg]) * row_bytes;
#pragma unroll
                for (int m = 0; m < NI; m++)
                    if (gval[m]) lds_dma16(row + goff[m], ring + (u * NI + m) * 1024);
            }
        }
    };
    issue(0);

    q8k_input<64 * NW>(x, nrm, K, wv, NW, lane, qtmp, bst, d8);
    __syncthreads();
    for (int t = threadIdx.x; t < ntask; t += 64 * NW)
        F::build_task(xq + (size_t)t * F::kDw, qtmp + 64 * (t >> 2), bst + 16 * (t >> 2), t & 3);
    __syncthreads();  // the prep region becomes the per-wave record area
    if (nrows == 0) return;

    // record sets: [pair half][slot][block] x 10 dwords
    uint32_t *rec = (uint32_t *)(lds + L.region) + (size_t)wv * NT * R * nblk * 10;
    const typename F::LC c = F::lane_consts(lane);
    typename F::XS xs0;
    if (T == 1 && lane < ntask) F::load_x(xs0, xq, lane);

    int slot = 0;
    bool stored = false;  // the epilogue stores were issued after the current row's loads
    for (int i = 0; i < nrows; i++) {
        const int row = wave + i * nwave;
        if constexpr (PRIO) set_prio((wv / 4 + i) % (NW / 4));  // as gemv_stream_kernel's PRIO
        if (stored)
            wait_vm<NT == 2 ? 3 : 1>();
        else
            wait_vm<0>();
        // read only by lanes with a task: no zero fill
        typename F::Frag f[NT][T];
#pragma unroll
        for (int u = 0; u < NT; u++)
#pragma unroll
            for (int tt = 0; tt < T; tt++) {
                const int t = lane + 64 * tt;
                if (t < ntask) f[u][tt] = St::frag(ring + u * NI * 1024 + (t >> 2) * St::BP, c);
            }
        // the slot's LDS reads have returned before the next row lands in it
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        issue(i + 1);
        stored = false;
#pragma unroll
        for (int u = 0; u < NT; u++)
#pragma unroll
            for (int tt = 0; tt < T; tt++) {
                const int t = lane + 64 * tt;
                int Ssum[8] = {0, 0, 0, 0, 0, 0, 0, 0}, M = 0;
                uint32_t h = 0;
                if (t < ntask) {
                    if (T == 1) {
                        F::dot(f[u][tt], xs0, c, Ssum, M);
                    } else {
                        typename F::XS xs;
                        F::load_x(xs, xq, t);
                        F::dot(f[u][tt], xs, c, Ssum, M);
                    }
                    h = F::hdr(f[u][tt]);
                }
                // the four tasks of a block are one lane quad: sum them
#pragma unroll
                for (int k = 0; k < 8; k++) Ssum[k] = group4_sum_i(Ssum[k]);
                if (F::kMin) M = group4_sum_i(M);
                if (t < ntask) {
                    const int q = t & 3;
                    uint32_t *r = rec + (((size_t)u * R + slot) * nblk + (t >> 2)) * 10;
                    r[2 * q] = (uint32_t)Ssum[2 * q];
                    r[2 * q + 1] = (uint32_t)Ssum[2 * q + 1];
                    if (q == 0) {
                        r[8] = (uint32_t)M;
                        r[9] = h;
                    }
                }
            }
        slot++;
        if (slot == R || i + 1 == nrows) {
            // epilogue (quants.rs:343-358 / :402-411), as gemv_q8k_kernel:
            // lane (r, k) replays sums[k] += d*sumi[k] over the blocks in
            // order (k = 0 also sumf -= dmin*minsum), then
            // s = sumf + sums[0] + ... + sums[7]
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int u = 0; u < NT; u++)
                q8k_fold<F::kMin>(rec + (size_t)u * R * nblk * 10, nblk * 10, d8, slot, 0, nblk, lane);
            __builtin_amdgcn_wave_barrier();
            const int r = lane >> 3, k = lane & 7;
            float out[NT];
#pragma unroll
            for (int u = 0; u < NT; u++) {
                float sums = 0.0f, sumf = 0.0f;
                if (r < slot) q8k_replay<F::kMin>(rec + ((size_t)(u * R + r)) * nblk * 10, nblk, k, sums, sumf);
                // Q6_K: sumf stays 0.0f, matching `let mut s = 0.0f32`; lane k = 0 holds it
                const float sv = group8_chain_first(sumf, sums);
                out[u] = sv;
            }
            if (k == 0 && r < slot) {  // lane 0 always stores: NT == 1: one store, else three
                const int Rr = row - (slot - 1 - r) * nwave, so = MULTI ? seg_of(Sg, Rr) : 0;
                if (PAIR) {
                    Sg.y[0][Rr] = out[0];
                    Sg.y[1][Rr] = out[NT - 1];
                    Sg.y[2][Rr] = swiglu1(out[0], out[NT - 1]);
                } else {
                    Sg.y[so][Rr - Sg.start[so]] = out[0];
                    if (!MULTI && Sg.ysum) Sg.ysum[Rr] = __fadd_rn(Sg.add[Rr], out[0]);
                }
            }
            __builtin_amdgcn_wave_barrier();
            stored = true;
            slot = 0;
        }
    }
}

// K-split variant for 4096 < K <= 20480 (one tensor, bit-exact; 2-5 slices
// when the layout fits the CU's LDS): the
// workgroup's waves are KS slices x NG row groups. A wave streams its slice
// (16 blocks) of its group's rows through its own ring slot and keeps its
// lane's x record in VGPRs; the slice's block records go to the group's
// shared record area. Every R rows all waves meet at a barrier, the slice-0
// wave of each group runs the reference-order epilogue over the 48 (K/256)
// blocks, and a second barrier frees the records. Every wave runs the
// workgroup's largest row count, so all reach the same barriers.
template <class F, int KS, int NG>
__global__ __launch_bounds__(64 * KS * NG) void gemv_q8k_ks_kernel(const Segs Sg, size_t row_bytes, int K,
                                                                  const float *__restrict__ x) {
    using St = Stage<typename Q8Base<F>::T>;
    constexpr int NW = KS * NG;
    constexpr int NI = (16 * St::BC + 63) / 64;  // 1 KB loads per slice
    extern __shared__ __align__(16) uint8_t lds[];
    const int nblk = K >> 8, ntask = 4 * nblk;
    const Q8SLayout L = q8k_stream_layout<F>(K, NG, NI * KS);  // records per group, ring per wave
    const int R = L.R;
    uint32_t *xq = (uint32_t *)(lds + L.xq);
    float *d8 = (float *)(lds + L.d8);
    uint32_t *qtmp = (uint32_t *)(lds + L.region);
    int *bst = (int *)(lds + L.region + K);
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sl = wv % KS, gi = wv / KS;
    const int t = 64 * sl + lane;  // this lane's task
    const bool act = t < ntask;
    const int G = blockIdx.x * NG + gi, nG = gridDim.x * NG;
    const int N = Sg.start[Sg.n];
    const int nrows = G < N ? (N - 1 - G) / nG + 1 : 0;
    const int G0 = blockIdx.x * NG;
    const int nmax = G0 < N ? (N - 1 - G0) / nG + 1 : 0;  // rows of the workgroup's first group
    const int nch = (min(nblk, 16 * sl + 16) - 16 * sl) * St::BC;  // chunks of this slice
    uint8_t *ring = lds + L.ring + (size_t)wv * NI * 1024;

    uint32_t goff[NI];
    bool gval[NI];
#pragma unroll
    for (int m = 0; m < NI; m++) {
        const int k = lane + 64 * m, b = k / St::BC;
        gval[m] = k < nch;
        goff[m] = (uint32_t)((16 * sl + b) * St::BB + 16 * (k - b * St::BC));
    }
    auto issue = [&](int i) {
        if (i < nrows) {  // wave-uniform
            const uint8_t *row = Sg.w[0] + (size_t)(G + i * nG) * row_bytes;
#pragma unroll
            for (int m = 0; m < NI; m++)
                if (gval[m]) lds_dma16(row + goff[m], ring + m * 1024);
        }
    };
    issue(0);

    quantize_blocks_lds(x, wv, NW, nblk, lane, qtmp, bst, d8);
    __syncthreads();
    for (int q = threadIdx.x; q < ntask; q += 64 * NW)
        F::build_task(xq + (size_t)q * F::kDw, qtmp + 64 * (q >> 2), bst + 16 * (q >> 2), q & 3);
    __syncthreads();  // the prep region becomes the record area
    if (nmax == 0) return;  // the whole workgroup: no rows

    uint32_t *rec = (uint32_t *)(lds + L.region) + (size_t)gi * R * nblk * 10;  // [slot][block] x 10
    const typename F::LC c = F::lane_consts(lane);
    typename F::XS xs0;
    if (act) F::load_x(xs0, xq, t);

    int slot = 0;
    bool stored = false;  // this wave's epilogue store came after its current row's loads
    for (int i = 0; i < nmax; i++) {
        if (i < nrows) {  // wave-uniform
            if (stored)
                wait_vm<1>();
            else
                wait_vm<0>();
            typename F::Frag f;
            if (act) f = St::frag(ring + (lane >> 2) * St::BP, c);
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue(i + 1);
            stored = false;
            int Ssum[8] = {0, 0, 0, 0, 0, 0, 0, 0}, M = 0;
            uint32_t h = 0;
            if (act) {
                F::dot(f, xs0, c, Ssum, M);
                h = F::hdr(f);
            }
#pragma unroll
            for (int k = 0; k < 8; k++) Ssum[k] = group4_sum_i(Ssum[k]);
            if (F::kMin) M = group4_sum_i(M);
            if (act) {
                const int q = t & 3;
                uint32_t *r = rec + ((size_t)slot * nblk + (t >> 2)) * 10;
                r[2 * q] = (uint32_t)Ssum[2 * q];
                r[2 * q + 1] = (uint32_t)Ssum[2 * q + 1];
                if (q == 0) {
                    r[8] = (uint32_t)M;
                    r[9] = h;
                }
            }
        }
        slot++;
        if (slot == R || i + 1 == nmax) {
            const int nr = min(slot, nrows - (i + 1 - slot));  // rows of this group in the batch
            // each slice folds the block factors into its own records
            __builtin_amdgcn_wave_barrier();
            if (nr > 0) q8k_fold<F::kMin>(rec, nblk * 10, d8, nr, 16 * sl, min(nblk, 16 * sl + 16), lane);
            __syncthreads();  // every slice's records of these rows are written
            if (sl == 0 && nr > 0) {
                // epilogue (quants.rs:343-358 / :402-411), as gemv_q8k_kernel
                const int r = lane >> 3, k = lane & 7;
                float sums = 0.0f, sumf = 0.0f;
                if (r < nr) q8k_replay<F::kMin>(rec + (size_t)(r) * nblk * 10, nblk, k, sums, sumf);
                // Q6_K: sumf stays 0.0f, matching `let mut s = 0.0f32`; lane k = 0 holds it
                const float sv = group8_chain_first(sumf, sums);
                if (k == 0 && r < nr) {  // lane 0 always stores: one store instruction
                    const int Rr = G + (i + 1 - slot + r) * nG;
                    Sg.y[0][Rr] = sv;
                    if (Sg.ysum) Sg.ysum[Rr] = __fadd_rn(Sg.add[Rr], sv);
                }
                stored = true;
            }
            __syncthreads();  // the records are free again
            slot = 0;
        }
    }
}

// Any K (multiple of 256) the fast kernel cannot hold: one thread per row
// running the reference loop verbatim on the workgroup's Q8_K blocks.
__global__ __launch_bounds__(TPB) void gemv_q8k_generic_kernel(uq_dtype dt, const uint8_t *__restrict__ W,
                                                               size_t row_bytes, int K, int N,
                                                               const float *__restrict__ x,
                                                               float *__restrict__ y,
                                                               const float *__restrict__ add,
                                                               float *__restrict__ ysum) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int nblk = K >> 8;
    uint32_t *q = (uint32_t *)lds;
    int *bs = (int *)(lds + K);
    float *d8 = (float *)(lds + K + (K / 16) * 4);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    quantize_blocks_lds(x, wid, WAVES, nblk, lane, q, bs, d8);
    __syncthreads();
    const int8_t *qs = (const int8_t *)q;
    for (int row = blockIdx.x * TPB + threadIdx.x; row < N; row += gridDim.x * TPB) {
        const uint8_t *Rw = W + (size_t)row * row_bytes;
        float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0}, sumf = 0.0f;
        for (int b = 0; b < nblk; b++) {
            int sumi[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            const int8_t *q8 = qs + 256 * b;
            if (dt == UQ_Q4_K) {
                const uint8_t *blk = Rw + (size_t)b * BQ4K;
                const uint8_t *s = blk + 4;
                int sc[8], m[8];
                for (int g = 0; g < 8; g++) {
                    if (g < 4) {
                        sc[g] = s[g] & 63;
                        m[g] = s[g + 4] & 63;
                    } else {
                        sc[g] = (s[g + 4] & 0xF) | ((s[g - 4] >> 6) << 4);
                        m[g] = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
                    }
                }
                for (int e = 0; e < 256; e++) {
                    const int pos = e % 64;
                    const uint8_t byte = blk[16 + 32 * (e / 64) + pos % 32];
                    const int a = pos < 32 ? (byte & 0xF) : (byte >> 4);
                    sumi[e % 8] += sc[e / 32] * a * q8[e];
                }
                const float d = __fmul_rn(d8[b], f16_bits_exact(blk[0] | (blk[1] << 8)));
                for (int k = 0; k < 8; k++) sums[k] = __fadd_rn(sums[k], __fmul_rn(d, (float)sumi[k]));
                int minsum = 0;
                for (int g = 0; g < 16; g++) minsum += bs[16 * b + g] * m[g / 2];
                const float dmin = __fmul_rn(f16_bits_exact(blk[2] | (blk[3] << 8)), d8[b]);
                sumf = __fsub_rn(sumf, __fmul_rn(dmin, (float)minsum));
            } else {
                const uint8_t *blk = Rw + (size_t)b * BQ6K;
                for (int e = 0; e < 256; e++) {
                    const int pos = e % 128;
                    const uint8_t byte = blk[64 * (e / 128) + pos % 64];
                    const int nib = pos < 64 ? (byte & 0xF) : (byte >> 4);
                    const int hi2 = (blk[128 + 32 * (e / 128) + pos % 32] >> (2 * (pos / 32))) & 3;
                    sumi[e % 8] += (int)(int8_t)blk[192 + e / 16] * ((nib | (hi2 << 4)) - 32) * q8[e];
                }
                const float d = __fmul_rn(d8[b], f16_bits_exact(blk[208] | (blk[209] << 8)));
                for (int k = 0; k < 8; k++) sums[k] = __fadd_rn(sums[k], __fmul_rn(d, (float)sumi[k]));
            }
        }
        float s = sumf;
        for (int k = 0; k < 8; k++) s = __fadd_rn(s, sums[k]);
        y[row] = s;
        if (ysum) ysum[row] = __fadd_rn(add[row], s);
    }
}

constexpr int UQ_Q8K_STREAM = 1;
// waves per workgroup of the streaming q8k kernel: the head's shapes for
// K <= 4096; fewer waves for the longer rows of K <= 12288 (LDS ring)
template <class F, int T> struct Q8SShape { static constexpr int NW = StreamShape<typename Q8Base<F>::T>::NW; };
template <> struct Q8SShape<Q6KQ8, 2> { static constexpr int NW = 8; };
template <> struct Q8SShape<Q6KQ8, 3> { static constexpr int NW = 8; };
template <> struct Q8SShape<Q4KQ8, 2> { static constexpr int NW = 12; };
template <> struct Q8SShape<Q4KQ8, 3> { static constexpr int NW = 12; };

template <class F, int T, bool MULTI>
bool q8k_stream_fits(int K) {
    using St = Stage<typename Q8Base<F>::T>;
    constexpr int NW = Q8SShape<F, T>::NW, NI = (16 * T * St::BC + 63) / 64;
    const Q8SLayout L = q8k_stream_layout<F>(K, NW, NI);
    return L.R > 0 && L.total <= kQ8SLds;
}

template <class F, int T, bool MULTI>
hipError_t launch_q8k_stream(const Segs &S, size_t row_bytes, int K, const float *x, hipStream_t s,
                             const RowNorm &nrm = RowNorm()) {
    using St = Stage<typename Q8Base<F>::T>;
    constexpr int NW = Q8SShape<F, T>::NW, NI = (16 * T * St::BC + 63) / 64;
    const int N = S.start[S.n];
    const Q8SLayout L = q8k_stream_layout<F>(K, NW, NI);
    const void *k = (const void *)gemv_q8k_stream_kernel<F, T, NW, MULTI>;
    const hipError_t e = allow_lds(k, L.total);
    if (e != hipSuccess) return e;
    const int grid = resident_grid(k, L.total, N, NW);
    if constexpr (!MULTI) {
        if ((N + grid * NW - 1) / (grid * NW) >= kPrioRows) {  // rows per wave
            const void *kp = (const void *)gemv_q8k_stream_kernel<F, T, NW, false, false, true>;
            const hipError_t ep = allow_lds(kp, L.total);
            if (ep != hipSuccess) return ep;
            hipLaunchKernelGGL((gemv_q8k_stream_kernel<F, T, NW, false, false, true>), dim3(grid), dim3(64 * NW),
                               L.total, s, S, row_bytes, K, x, nrm);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((gemv_q8k_stream_kernel<F, T, NW, MULTI>), dim3(grid), dim3(64 * NW), L.total, s, S,
                       row_bytes, K, x, nrm);
    return hipGetLastError();
}

template <class F>
hipError_t launch_q8k_pair(const Segs &S, size_t row_bytes, int K, const float *x, hipStream_t s, bool *done,
                           const RowNorm &nrm = RowNorm()) {
    using St = Stage<typename Q8Base<F>::T>;
    constexpr int NW = UQ_STREAM_PAIR_NW, NI = (16 * St::BC + 63) / 64;
    *done = false;
    const Q8SLayout L = q8k_stream_layout<F>(K, NW, NI, 2);
    if (!UQ_Q8K_STREAM || F::ntasks(K) > 64 || L.R == 0 || L.total > kQ8SLds) return hipSuccess;
    const int N = S.start[S.n];
    const void *k = (const void *)gemv_q8k_stream_kernel<F, 1, NW, false, true>;
    const hipError_t e = allow_lds(k, L.total);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((gemv_q8k_stream_kernel<F, 1, NW, false, true>), dim3(resident_grid(k, L.total, N, NW)),
                       dim3(64 * NW), L.total, s, S, row_bytes, K, x, nrm);
    *done = true;
    return hipGetLastError();
}

template <class F>
hipError_t launch_q8k_ks(const Segs &S, size_t row_bytes, int K, const float *x, hipStream_t s, bool *done) {
    using St = Stage<typename Q8Base<F>::T>;
    constexpr int NI = (16 * St::BC + 63) / 64;
    const int ks = (F::ntasks(K) + 63) / 64;
    *done = false;
    auto go = [&](auto kern, int KSv, int NGv) -> hipError_t {
        const Q8SLayout L = q8k_stream_layout<F>(K, NGv, NI * KSv);
        if (L.R == 0 || L.total > kQ8SLds) return hipSuccess;
        const int N = S.start[S.n];
        const void *k = (const void *)kern;
        hipError_t e = allow_lds(k, L.total);
        if (e != hipSuccess) return e;
        // one workgroup per CU, NG row groups each, rows dealt round-robin to the groups
        const int rpg = (N + num_cus() * NGv - 1) / (num_cus() * NGv);  // rows per group
        const int grid = (N + rpg * NGv - 1) / (rpg * NGv);
        hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * KSv * NGv), L.total, s, S, row_bytes, K, x);
        *done = true;
        return hipGetLastError();
    };
    if (ks == 2) return go(gemv_q8k_ks_kernel<F, 2, 6>, 2, 6);
    if (ks == 3) return go(gemv_q8k_ks_kernel<F, 3, 4>, 3, 4);
    if (ks == 4) return go(gemv_q8k_ks_kernel<F, 4, 3>, 4, 3);
    if (ks == 5) return go(gemv_q8k_ks_kernel<F, 5, 3>, 5, 3);
    return hipSuccess;
}

template <class F, bool MULTI>
hipError_t launch_q8k_fast_m(const Segs &S, size_t row_bytes, int K, const float *x, hipStream_t s) {
    const int N = S.start[S.n];
    const Q8KLayout L = q8k_layout<F>(K);
    if (UQ_Q8K_STREAM && !MULTI && F::ntasks(K) > 64 && F::ntasks(K) <= 320) {
        bool done = false;
        const hipError_t e = launch_q8k_ks<F>(S, row_bytes, K, x, s, &done);
        if (e != hipSuccess || done) return e;
    }
    if (UQ_Q8K_STREAM) {
        const int T = (F::ntasks(K) + 63) / 64;  // tasks per lane
        if (T == 1 && q8k_stream_fits<F, 1, MULTI>(K)) return launch_q8k_stream<F, 1, MULTI>(S, row_bytes, K, x, s);
        if (T == 2 && q8k_stream_fits<F, 2, MULTI>(K)) return launch_q8k_stream<F, 2, MULTI>(S, row_bytes, K, x, s);
        if (T == 3 && q8k_stream_fits<F, 3, MULTI>(K)) return launch_q8k_stream<F, 3, MULTI>(S, row_bytes, K, x, s);
    }
    if (F::ntasks(K) <= 64) {
        const void *k = (const void *)gemv_q8k_kernel<F, true, MULTI>;
        hipLaunchKernelGGL((gemv_q8k_kernel<F, true, MULTI>), dim3(resident_grid(k, L.total, N)), dim3(TPB), L.total,
                           s, S, row_bytes, K, x);
    } else {
        const void *k = (const void *)gemv_q8k_kernel<F, false, MULTI>;
        hipLaunchKernelGGL((gemv_q8k_kernel<F, false, MULTI>), dim3(resident_grid(k, L.total, N)), dim3(TPB),
                           L.total, s, S, row_bytes, K, x);
    }
    return hipGetLastError();
}

// gemv_quant_q8k over a segment table (all segments share dtype and K).
hipError_t launch_q8k_segs(uq_dtype dt, int K, size_t row_bytes, const Segs &S, const float *x, hipStream_t s) {
    if (S.start[S.n] == 0) return hipSuccess;
    const bool multi = S.n > 1;
    if (dt == UQ_Q4_K && q8k_layout<Q4KQ8>(K).total <= kLdsCap)
        return multi ? launch_q8k_fast_m<Q4KQ8, true>(S, row_bytes, K, x, s)
                     : launch_q8k_fast_m<Q4KQ8, false>(S, row_bytes, K, x, s);
    if (dt == UQ_Q6_K && q8k_layout<Q6KQ8>(K).total <= kLdsCap)
        return multi ? launch_q8k_fast_m<Q6KQ8, true>(S, row_bytes, K, x, s)
                     : launch_q8k_fast_m<Q6KQ8, false>(S, row_bytes, K, x, s);
    const size_t lds = (size_t)K + (size_t)(K / 16) * 4 + (size_t)(K / 256) * 4;
    if (lds > kLdsCap) return hipErrorInvalidValue;
    for (int i = 0; i < S.n; i++) {
        const int N = S.start[i + 1] - S.start[i];
        if (N == 0) continue;
        int grid = (N + TPB - 1) / TPB;
        if (grid > num_cus() * 4) grid = num_cus() * 4;
        hipLaunchKernelGGL(gemv_q8k_generic_kernel, dim3(grid), dim3(TPB), lds, s, dt, S.w[i], row_bytes, K, N, x,
                           S.y[i], S.n == 1 ? S.add : nullptr, S.n == 1 ? S.ysum : nullptr);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

Segs batch_segs(const WeightsView *w, int n, float *const *y) {
    Segs S{};
    S.n = n;
    S.start[0] = 0;
    for (int i = 0; i < n; i++) {
        S.w[i] = w[i].bytes;
        S.w2[i] = nullptr;
        S.y[i] = y[i];
        S.start[i + 1] = S.start[i] + w[i].dim_out;
    }
    return S;
}

}  // namespace

hipError_t launch_gemv(const WeightsView &w, const float *x, float *y, hipStream_t s) {
    return launch_segs(w.dtype, w.dim_in, w.row_bytes, one_seg(w, nullptr, y), false, x, s);
}

hipError_t launch_gemv_batch(const WeightsView *w, int n, const float *x, float *const *y, hipStream_t s) {
    static_assert(kMaxSegs == UQ_GEMV_BATCH_MAX, "segment table size");
    return launch_segs(w[0].dtype, w[0].dim_in, w[0].row_bytes, batch_segs(w, n, y), false, x, s);
}

hipError_t launch_gemv_q8k_batch(const WeightsView *w, int n, const float *x, float *const *y, hipStream_t s) {
    return launch_q8k_segs(w[0].dtype, w[0].dim_in, w[0].row_bytes, batch_segs(w, n, y), x, s);
}

hipError_t launch_gate_up_swiglu(const WeightsView &g, const WeightsView &u, const float *x, float *h,
                                 hipStream_t s) {
    return launch_segs(g.dtype, g.dim_in, g.row_bytes, one_seg(g, u.bytes, h), true, x, s);
}

// g = gemv_quant_q8k(gate, x), u = gemv_quant_q8k(up, x) and h = swiglu(g, u)
// in one launch; *done is false when the shapes do not take the streaming
// kernel (the caller then runs the three steps).
hipError_t launch_q8k_gate_up(const WeightsView &g, const WeightsView &u, const float *x, float *yg, float *yu,
                              float *h, hipStream_t s, bool *done) {
    *done = false;
    if (g.dim_out == 0) {
        *done = true;
        return hipSuccess;
    }
    Segs S{};
    S.n = 1;
    S.start[0] = 0;
    S.start[1] = g.dim_out;
    S.w[0] = g.bytes;
    S.w2[0] = u.bytes;
    S.y[0] = yg;
    S.y[1] = yu;
    S.y[2] = h;
    if (g.dtype == UQ_Q4_K) return launch_q8k_pair<Q4KQ8>(S, g.row_bytes, g.dim_in, x, s, done);
    if (g.dtype == UQ_Q6_K) return launch_q8k_pair<Q6KQ8>(S, g.row_bytes, g.dim_in, x, s, done);
    return hipSuccess;
}

hipError_t launch_gemv_q8k(const WeightsView &w, const float *x, float *y, hipStream_t s) {
    return launch_q8k_segs(w.dtype, w.dim_in, w.row_bytes, one_seg(w, nullptr, y), x, s);
}

namespace {
// The streaming kernel with one task per lane (K <= 4096), the one launch
// shape that forms a row norm in its prologue.
template <class F, bool MULTI>
hipError_t q8k_norm_stream(const Segs &S, size_t row_bytes, int K, const float *x, const RowNorm &nrm,
                           hipStream_t s, bool *done) {
    *done = false;
    if (!UQ_Q8K_STREAM || F::ntasks(K) > 64 || !q8k_stream_fits<F, 1, MULTI>(K)) return hipSuccess;
    *done = true;
    return launch_q8k_stream<F, 1, MULTI>(S, row_bytes, K, x, s, nrm);
}
}  // namespace

hipError_t launch_gemv_q8k_batch_norm(const WeightsView *w, int n, const float *x, float *const *y, const RowNorm &nrm,
                                      hipStream_t s, bool *done) {
    *done = false;
    const Segs S = batch_segs(w, n, y);
    if (S.start[S.n] == 0 || w[0].dim_in == 0) return hipSuccess;
    const int K = w[0].dim_in;
    const size_t rb = w[0].row_bytes;
    if (w[0].dtype == UQ_Q4_K)
        return n > 1 ? q8k_norm_stream<Q4KQ8, true>(S, rb, K, x, nrm, s, done)
                     : q8k_norm_stream<Q4KQ8, false>(S, rb, K, x, nrm, s, done);
    if (w[0].dtype == UQ_Q6_K)
        return n > 1 ? q8k_norm_stream<Q6KQ8, true>(S, rb, K, x, nrm, s, done)
                     : q8k_norm_stream<Q6KQ8, false>(S, rb, K, x, nrm, s, done);
    return hipSuccess;
}

hipError_t launch_q8k_gate_up_norm(const WeightsView &g, const WeightsView &u, const float *x, float *yg, float *yu,
                                   float *h, const RowNorm &nrm, hipStream_t s, bool *done) {
    *done = false;
    if (g.dim_out == 0 || g.dim_in == 0) return hipSuccess;
    Segs S{};
    S.n = 1;
    S.start[0] = 0;
    S.start[1] = g.dim_out;
    S.w[0] = g.bytes;
    S.w2[0] = u.bytes;
    S.y[0] = yg;
    S.y[1] = yu;
    S.y[2] = h;
    if (g.dtype == UQ_Q4_K) return launch_q8k_pair<Q4KQ8>(S, g.row_bytes, g.dim_in, x, s, done, nrm);
    if (g.dtype == UQ_Q6_K) return launch_q8k_pair<Q6KQ8>(S, g.row_bytes, g.dim_in, x, s, done, nrm);
    return hipSuccess;
}

hipError_t launch_gemv_q8k_sum(const WeightsView &w, const float *x, float *y, const float *add, float *ysum,
                               hipStream_t s) {
    Segs S = one_seg(w, nullptr, y);
    S.add = add;
    S.ysum = ysum;
    return launch_q8k_segs(w.dtype, w.dim_in, w.row_bytes, S, x, s);
}

// Dynamic LDS above 64 KB must be allowed per kernel and device, once.
hipError_t allow_lds(const void *kernel, size_t lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    static std::mutex mu;
    static std::map<std::pair<const void *, int>, size_t> done;
    std::lock_guard<std::mutex> g(mu);
    size_t &have = done[{kernel, dev}];
    if (have >= lds) return hipSuccess;
    RelaxedCapture relax;
    e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e == hipSuccess) have = lds;
    return e;
}

}  // namespace uq
