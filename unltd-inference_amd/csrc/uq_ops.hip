// Per-layer non-linear kernels of the forward (crates/unltd-tensor/src/
// kernels.rs), on device so activations stay in HBM between layers. Each
// kernel follows the reference's arithmetic step for step: f32 steps as
// separate IEEE operations (built -ffp-contract=off, with explicit _rn
// intrinsics where the order matters), f64 sums in the reference's order.
//
// Sequential f64 sums (rmsnorm, l2_norm_rows) are formed as a tree sum S
// plus a rigorous bound: for n non-negative terms the sequential sum and S
// both lie within (n + log2 n + 2) * 2^-53 * S of the exact sum, so when
// both ends of [S - e, S + e] round to the same f32 result (rounding is
// monotonic), that is the reference's result. Otherwise (probability about
// n * 2^-29 per row) one wave replays the sequential loop.
//
// Transcendentals: f32 exp / log are evaluated in f64 and rounded once
// (correctly rounded but for rare near-midpoint arguments), and the rope
// angles use the f64 sin / cos of the device library; the reference uses
// the platform libm, so those results agree within about 1 ulp.
#include "uq_device.h"
#include "uq_internal.h"
#include "uq_q8k_quant.h"

namespace uq {

namespace {

constexpr int OPS_TPB = 256;

__device__ __forceinline__ float logf_cr(float v) { return (float)log((double)v); }

__device__ float block_max_f(float v, float *red) {
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) t = fmaxf(t, red[i]);
    __syncthreads();
    return t;
}

// sigmoid (kernels.rs:198-203), silu (:207-212), softplus (:217-228)
__device__ __forceinline__ float sigmoid1(float v) { return __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_cr(-v))); }
__device__ __forceinline__ float silu1(float v) { return __fdiv_rn(v, __fadd_rn(1.0f, expf_cr(-v))); }
__device__ __forceinline__ float softplus1(float v) { return v > 20.0f ? v : logf_cr(__fadd_rn(1.0f, expf_cr(v))); }

// rmsnorm (kernels.rs:61-78), one workgroup per row of n; rows xs (input)
// and ys (output) floats apart. Two fusions of the layer forward: with xb
// the row normalised is x + xb (an f32 add), also written to xsum (the
// residual and the norm after it, qwen35_forward.rs:525-530); with z the
// output is multiplied by silu(z) (the gated norm, :495-511; z in the
// output's layout). Q8 (PT * TPB >= n, n a multiple of 256): the outputs
// also go to LDS and each wave quantizes 256-blocks of them into the q8k
// GEMM's planes q8 (q8k_quantize_wave, as the GEMM's prep would from the
// stored rows: the same f32 values); workgroups rows .. q8.Mp - 1 write the
// padding rows' all-zero blocks. PT > 0 (n <= PT * TPB): a thread's elements are
// loaded once, all before the sum, and kept in registers. Rows up to 4096
// run on 1024 threads (four elements each: the per-thread chains of loads
// and f64 adds are a quarter as long; 3.2 us per 4096-row in a graph against
// 5.0 us on 256 threads).
template <int PT, int TPB = OPS_TPB, bool Q8 = false>
__global__ __launch_bounds__(TPB) void rmsnorm_kernel(float *__restrict__ out, const float *__restrict__ x,
                                                      const float *__restrict__ w, int n, float eps, int xs,
                                                      int ys, const float *__restrict__ xb,
                                                      float *__restrict__ xsum, const float *__restrict__ z,
                                                      Q8Planes q8 = {}, int rows = 0, bool q6 = false) {
    __shared__ double red[TPB / 64];
    __shared__ float bc;
    constexpr int QE = Q8 ? PT * TPB : 1, QW = Q8 ? TPB / 64 : 1;
    __shared__ float yq[QE];
    __shared__ int8_t qsw[QW][256];
    __shared__ int bsw[QW][16];
    const int lane = threadIdx.x & 63, wq = threadIdx.x >> 6;
    auto quantize = [&](int b, const float (&v)[4]) {
        if (q6)
            q8k_quantize_wave<true>(v, lane, qsw[wq], bsw[wq], q8, blockIdx.x, b);
        else
            q8k_quantize_wave<false>(v, lane, qsw[wq], bsw[wq], q8, blockIdx.x, b);
    };
    if constexpr (Q8) {
        if ((int)blockIdx.x >= rows) {  // a padding row of the planes
            const float v0[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int b = wq; b < n / 256; b += TPB / 64) quantize(b, v0);
            return;
        }
    }
    const float *xr = x + (size_t)blockIdx.x * xs;
    const float *xbr = xb ? xb + (size_t)blockIdx.x * xs : nullptr;
    float *yr = out + (size_t)blockIdx.x * ys;
    auto val = [&](int i) { return xbr ? __fadd_rn(xr[i], xbr[i]) : xr[i]; };
    constexpr int R = PT > 0 ? PT : 1;
    float v[R], wv[R], zv[R];
    double s = 0.0;
    if constexpr (PT > 0) {
        // the weights and z are loaded with x, before the sum
#pragma unroll
        for (int k = 0; k < PT; k++) {
            const int i = threadIdx.x + k * TPB;
            v[k] = i < n ? val(i) : 0.0f;
            wv[k] = i < n ? w[i] : 0.0f;
            zv[k] = (z && i < n) ? z[(size_t)blockIdx.x * ys + i] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < PT; k++) {
            const int i = threadIdx.x + k * TPB;
            if (i < n) {
                if (xsum) xsum[(size_t)blockIdx.x * xs + i] = v[k];
                s += (double)__fmul_rn(v[k], v[k]);
            }
        }
    } else {
        for (int i = threadIdx.x; i < n; i += TPB) {
            const float t = val(i);
            if (xsum) xsum[(size_t)blockIdx.x * xs + i] = t;
            s += (double)__fmul_rn(t, t);
        }
    }
    const double S = block_sum_d<TPB>(s, red);
    const double dn = (double)n;
    const float mean = seq_sum_f32<TPB>(val, n, S, [dn](double u) { return (float)(u / dn); }, &bc);
    const float scale = __fdiv_rn(1.0f, sqrtf_cr(__fadd_rn(mean, eps)));
    auto emit = [&](int i, float t, float wi, float zi) {
        float y = __fmul_rn(__fmul_rn(t, scale), wi);
        if (z) y = __fmul_rn(y, silu1(zi));
        yr[i] = y;
        if constexpr (Q8) yq[i] = y;
    };
    if constexpr (PT > 0) {
#pragma unroll
        for (int k = 0; k < PT; k++) {
            const int i = threadIdx.x + k * TPB;
            if (i < n) emit(i, v[k], wv[k], zv[k]);
        }
    } else {
        for (int i = threadIdx.x; i < n; i += TPB)
            emit(i, val(i), w[i], z ? z[(size_t)blockIdx.x * ys + i] : 0.0f);
    }
    if constexpr (Q8) {
        static_assert(PT > 0, "the row is held in LDS");
        __syncthreads();  // every output in yq
        for (int b = wq; b < n / 256; b += TPB / 64) {
            const float4 f = *(const float4 *)(yq + 256 * b + 4 * lane);
            const float v[4] = {f.x, f.y, f.z, f.w};
            quantize(b, v);
        }
    }
}

// l2_norm_rows (kernels.rs:236-256), in place, one workgroup per row.
__global__ __launch_bounds__(OPS_TPB) void l2norm_kernel(float *__restrict__ data, int dim, float eps) {
    __shared__ double red[OPS_TPB / 64];
    __shared__ float bc;
    float *r = data + (size_t)blockIdx.x * dim;
    double s = 0.0;
    for (int i = threadIdx.x; i < dim; i += OPS_TPB) s += (double)__fmul_rn(r[i], r[i]);
    const double S = block_sum_d<OPS_TPB>(s, red);
    const float sum32 = seq_sum_f32<OPS_TPB>([r](int i) { return r[i]; }, dim, S, [](double v) { return (float)v; }, &bc);
    const float scale = __fdiv_rn(1.0f, fmaxf(sqrtf_cr(sum32), eps));
    for (int i = threadIdx.x; i < dim; i += OPS_TPB) r[i] = __fmul_rn(r[i], scale);
}

// Pairwise tree (kernels.rs:27-42) of lv[0, len) in LDS, level by level:
// pairs (2i, 2i+1), an odd tail carried up. Every thread takes part;
// returns lv[0] to all (len <= 2 * OPS_TPB * kTreeRegs).
constexpr int kTreeRegs = 16;
__device__ double lds_tree(double *lv, int len) {
    while (len > 1) {
        const int nl = (len + 1) / 2;
        double v[kTreeRegs];
        int c = 0;
        for (int p = threadIdx.x; p < nl; p += OPS_TPB, c++) v[c] = 2 * p + 1 < len ? lv[2 * p] + lv[2 * p + 1] : lv[2 * p];
        __syncthreads();
        c = 0;
        for (int p = threadIdx.x; p < nl; p += OPS_TPB, c++) lv[p] = v[c];
        __syncthreads();
        len = nl;
    }
    const double r = lv[0];
    __syncthreads();
    return r;
}

// softmax (kernels.rs:157-168), one workgroup per row, in place allowed.
// The denominator is pairwise_sum_f64 over the row. For a chunk size C that
// is a power of two, level log2(C) of that tree holds the trees of the full
// C-chunks followed by the tree of the remainder (whose node is always the
// carried odd tail below that level), so the row sum is the pairwise tree
// over the chunk sums: each chunk is reduced in LDS, then the chunk sums.
constexpr int kSmChunk = 2 * OPS_TPB * kTreeRegs;  // 8192
constexpr int kSmMaxChunks = 2048;
static_assert((kSmChunk & (kSmChunk - 1)) == 0, "chunk trees must be nodes of the row tree");
// Rows of token z = blockIdx.y (the attention of a prefill) are n + z dn
// long and start zst floats after token z - 1's.
__global__ __launch_bounds__(OPS_TPB) void softmax_kernel(float *out, const float *x, int n, float scale, int dn,
                                                          size_t zst) {
    __shared__ double lv[kSmChunk / 2];
    __shared__ double cs[kSmMaxChunks];
    __shared__ float red[OPS_TPB / 64];
    n += (int)blockIdx.y * dn;
    const size_t row0 = (size_t)blockIdx.y * zst + (size_t)blockIdx.x * n;
    const float *xr = x + row0;
    float *yr = out + row0;
    float m = -INFINITY;
    for (int i = threadIdx.x; i < n; i += OPS_TPB) m = fmaxf(m, xr[i]);
    m = block_max_f(m, red);
    auto ex = [&](int i) { return expf_cr(__fmul_rn(__fsub_rn(xr[i], m), scale)); };
    const int nch = (n + kSmChunk - 1) / kSmChunk;
    for (int c = 0; c < nch; c++) {
        const int base = c * kSmChunk, cl = min(kSmChunk, n - base);
        const int len = (cl + 1) / 2;  // level 1 straight from the exponentials
        for (int p = threadIdx.x; p < len; p += OPS_TPB) {
            const int i = base + 2 * p;
            lv[p] = 2 * p + 1 < cl ? (double)ex(i) + (double)ex(i + 1) : (double)ex(i);
        }
        __syncthreads();
        const double t = lds_tree(lv, len);
        if (threadIdx.x == 0) cs[c] = t;
    }
    __syncthreads();
    const double sum = lds_tree(cs, nch);
    for (int i = threadIdx.x; i < n; i += OPS_TPB) yr[i] = (float)((double)ex(i) / sum);
}

// softmax_kernel for rows of at most kSmWaveMax (the attention of a short
// context or of a prefill chunk): one wave per row, four rows a workgroup,
// no barrier. Lane l holds elements [16 l, 16 l + 16); the row's pairwise
// tree (kernels.rs:21-42) is the lanes' 16-element trees, then the wave's
// fixed tree over the lanes (wave_sum_d), with the missing elements as
// zeros: every term is an exponential (>= +0), so a zero added where the
// tree carries an odd tail up leaves the same value. Row r of token z =
// blockIdx.y (r < nr) is n + z dn long, token z's rows start zst floats
// after token z - 1's.
constexpr int kSmWaveMax = 1024;
__global__ __launch_bounds__(OPS_TPB) void softmax_wave_kernel(float *out, const float *x, int n, float scale, int dn,
                                                               size_t zst, int nr) {
    const int lane = threadIdx.x & 63, r = blockIdx.x * (OPS_TPB / 64) + (int)(threadIdx.x >> 6);
    if (r >= nr) return;  // the whole wave
    n += (int)blockIdx.y * dn;
    const size_t row0 = (size_t)blockIdx.y * zst + (size_t)r * n;
    const float *xr = x + row0;
    float *yr = out + row0;
    const int i0 = 16 * lane;
    float v[16];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        v[k] = i0 + k < n ? xr[i0 + k] : -INFINITY;
        m = fmaxf(m, v[k]);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
#pragma unroll
    for (int k = 0; k < 16; k++) v[k] = i0 + k < n ? expf_cr(__fmul_rn(__fsub_rn(v[k], m), scale)) : 0.0f;
    double t[8];
#pragma unroll
    for (int k = 0; k < 8; k++) t[k] = (double)v[2 * k] + (double)v[2 * k + 1];
#pragma unroll
    for (int w = 4; w >= 1; w >>= 1)
#pragma unroll
        for (int k = 0; k < w; k++) t[k] = t[2 * k] + t[2 * k + 1];
    const double sum = wave_sum_d(t[0]);
#pragma unroll
    for (int k = 0; k < 16; k++)
        if (i0 + k < n) yr[i0 + k] = (float)((double)v[k] / sum);
}

// sigmoid, silu, softplus, gelu_tanh (kernels.rs:185-194)
__global__ void unary_kernel(int op, const float *__restrict__ x, size_t n, float *__restrict__ out) {
    for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < n; t += (size_t)gridDim.x * blockDim.x) {
        const float v = x[t];
        float r;
        if (op == 0)
            r = sigmoid1(v);
        else if (op == 1)
            r = silu1(v);
        else if (op == 2)
            r = softplus1(v);
        else {  // gelu_tanh (kernels.rs:185-194), f64 left to right
            const double d = (double)v;
            const double inner = 0.7978845608028654 * (d + 0.044715 * d * d * d);
            r = (float)(0.5 * d * (1.0 + tanh(inner)));
        }
        out[t] = r;
    }
}

// ssm_conv (kernels.rs:265-305): out[t*channels + c], sequential f32 sum.
__global__ void ssm_conv_kernel(float *__restrict__ out, const float *__restrict__ x, const float *__restrict__ kern,
                                int d_conv, int channels, int n_t) {
    const size_t total = (size_t)n_t * channels;
    for (size_t o = blockIdx.x * (size_t)blockDim.x + threadIdx.x; o < total; o += (size_t)gridDim.x * blockDim.x) {
        const int t = (int)(o / channels), c = (int)(o % channels);
        float s = 0.0f;
        for (int tau = 0; tau < d_conv; tau++)
            s = __fadd_rn(s, __fmul_rn(x[(size_t)(t + tau) * channels + c], kern[(size_t)tau * channels + c]));
        out[o] = s;
    }
}

// One token of the GatedDeltaNet conv (qwen35_forward.rs:427-454), one
// thread per channel c: ssm_conv's sequential sum over the window's rows,
// with the kernel indexed as the GGUF tensor ssm_conv1d.weight is stored,
// [c][tau] (the forward transposes it first, :441-446), then silu of it,
// and the window's shift up by a row (:449-450).
__global__ void conv_step_kernel(float *__restrict__ win, const float *__restrict__ kern, float *__restrict__ raw,
                                 float *__restrict__ act, int d_conv, int channels) {
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < channels; c += gridDim.x * blockDim.x) {
        float x[9];
        for (int r = 0; r < d_conv; r++) x[r] = win[(size_t)r * channels + c];
        float s = 0.0f;
        for (int tau = 0; tau < d_conv; tau++) s = __fadd_rn(s, __fmul_rn(x[tau], kern[(size_t)c * d_conv + tau]));
        raw[c] = s;
        act[c] = silu1(s);
        for (int r = 1; r < d_conv; r++) win[(size_t)(r - 1) * channels + c] = x[r];
    }
}

// gdn_fused_step (kernels.rs:316-375), one workgroup per head, thread j
// owns column j of the head's dim x dim state: every step of the
// reference touches column j only through S[:, j], k, q, v[j], so the
// column is processed alone, with its f64 dots in the reference's order.
__global__ void gdn_step_kernel(float *__restrict__ state, float *__restrict__ out, const float *__restrict__ q,
                                const float *__restrict__ k, const float *__restrict__ v,
                                const float *__restrict__ gate, const float *__restrict__ beta, int dim,
                                float scale, int n_qk) {
    const int h = blockIdx.x, hq = h % n_qk;  // q/k head of v head h (qwen35_forward.rs:475)
    float *S = state + (size_t)h * dim * dim;
    const float *qh = q + (size_t)hq * dim, *kh = k + (size_t)hq * dim, *vh = v + (size_t)h * dim;
    const float g_exp = expf_cr(gate[h]), bt = beta[h];
    for (int j = threadIdx.x; j < dim; j += blockDim.x) {
        double sum = 0.0;
        for (int i = 0; i < dim; i++) {
            const float sv = __fmul_rn(S[(size_t)i * dim + j], g_exp);
            S[(size_t)i * dim + j] = sv;
            sum += (double)__fmul_rn(sv, kh[i]);
        }
        const float d = __fmul_rn(__fsub_rn(vh[j], (float)sum), bt);
        double o = 0.0;
        for (int i = 0; i < dim; i++) {
            const float sv = __fadd_rn(S[(size_t)i * dim + j], __fmul_rn(kh[i], d));
            S[(size_t)i * dim + j] = sv;
            o += (double)__fmul_rn(sv, qh[i]);
        }
        out[(size_t)h * dim + j] = __fmul_rn((float)o, scale);
    }
}

// The same step for dim <= 128 with the column in VGPRs: a workgroup of
// eight waves per 64 columns of a head, grid (dim / 64, heads); wave w holds
// rows [16w, 16w + 16) of the 64 columns, loaded once and stored once.
// Each f64 dot is the eight waves' partial sums (each in row order) added in
// LDS, plus a bound: any order of summing n terms lies within
// (n - 1) 2^-53 sum|t| of the exact sum, as does the reference's
// sequential loop, so when both ends of [S - e, S + e] round to one f32
// that is the reference's (float)sum. Otherwise (rarely; the decision is
// the same for every wave) the column goes through LDS and the loop runs in
// the reference's order.
constexpr int kGdnWaves = 8, kGdnRows = 16;  // waves per workgroup, rows per wave
__global__ __launch_bounds__(64 * kGdnWaves) void gdn_step_wg_kernel(float *__restrict__ state, float *__restrict__ out,
                                                         const float *__restrict__ q, const float *__restrict__ k,
                                                         const float *__restrict__ v, const float *__restrict__ gate,
                                                         const float *__restrict__ beta, int dim, float scale,
                                                         int n_qk) {
    __shared__ double ps[kGdnWaves][64], pa[kGdnWaves][64];
    __shared__ float col[128][64];  // the column, for the ordered replay
    __shared__ float kq[2][128];
    const int h = blockIdx.y, hq = h % n_qk, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int j = blockIdx.x * 64 + lane;
    const bool live = j < dim;
    const int i0 = kGdnRows * wv;
    float *S = state + (size_t)h * dim * dim + (live ? j : 0);
    // every global load first (state rows, v, gate, beta, k, q), one round trip
    float c[kGdnRows];
#pragma unroll
    for (int r = 0; r < kGdnRows; r++) c[r] = (i0 + r < dim && live) ? S[(size_t)(i0 + r) * dim] : 0.0f;
    const float vj = live ? v[(size_t)h * dim + j] : 0.0f, gh = gate[h], bt = beta[h];
    if (threadIdx.x < dim) {
        kq[0][threadIdx.x] = k[(size_t)hq * dim + threadIdx.x];
        kq[1][threadIdx.x] = q[(size_t)hq * dim + threadIdx.x];
    }
    __syncthreads();
    const float g_exp = expf_cr(gh);
#pragma unroll
    for (int r = 0; r < kGdnRows; r++) c[r] = __fmul_rn(c[r], g_exp);
    // (float) of the sequential f64 sum over i < dim of c_i * kq[sel][i]
    auto dot = [&](int sel) {
        double s = 0.0, a = 0.0;
#pragma unroll
        for (int r = 0; r < kGdnRows; r++)
            if (i0 + r < dim) {
                const double t = (double)__fmul_rn(c[r], kq[sel][i0 + r]);
                s += t;
                a += fabs(t);
            }
        ps[wv][lane] = s;
        pa[wv][lane] = a;
        __syncthreads();
        double S4 = 0.0, A4 = 0.0;
#pragma unroll
        for (int u = 0; u < kGdnWaves; u++) {
            S4 += ps[u][lane];
            A4 += pa[u][lane];
        }
        __syncthreads();  // ps / pa are free for the next dot
        const double e = (double)(dim + 66) * 0x1p-52 * A4;
        const float lo = (float)(S4 - e), hi = (float)(S4 + e);
        // one decision for the workgroup: any lane of any wave undecided
        const int undecided = __syncthreads_or(__float_as_uint(lo) != __float_as_uint(hi));
        if (!undecided) return lo;
#pragma unroll
        for (int r = 0; r < kGdnRows; r++)
            if (i0 + r < dim) col[i0 + r][lane] = c[r];
        __syncthreads();
        double qq = 0.0;
        for (int i = 0; i < dim; i++) qq += (double)__fmul_rn(col[i][lane], kq[sel][i]);
        __syncthreads();
        return (float)qq;
    };
    const float sum = dot(0);
    const float d = __fmul_rn(__fsub_rn(vj, sum), bt);
#pragma unroll
    for (int r = 0; r < kGdnRows; r++)
        if (i0 + r < dim) {
            c[r] = __fadd_rn(c[r], __fmul_rn(kq[0][i0 + r], d));
            if (live) S[(size_t)(i0 + r) * dim] = c[r];
        }
    const float o = dot(1);
    if (live && wv == 0) out[(size_t)h * dim + j] = __fmul_rn(o, scale);
}

// ---- the GatedDeltaNet prefill: the recurrent part of nt tokens ----------
// Of the step's work per token only the delta rule carries state from token
// to token; the conv over [window; qkv rows], silu, the q / k l2 norms and
// the gates of every token, and the gated rmsnorm of every output, are
// independent per token and run as row-parallel launches around the scan.

// Conv, silu and l2 norm of nt tokens (gdn_conv_norm_kernel per token),
// one wave per unit (b, t), four units a workgroup: for b < n_chunks the
// wave forms chunk b of token t into cv[t] (the q and k chunks normalised),
// lane l its channels l and l + 64 (hd <= 128); the window seen by token t
// is entries t .. t + d_conv - 1 of the sequence [win rows 0 .. d_conv - 2;
// qkv rows 0 .. nt - 1]. The norm's sum of squares is the wave's tree with
// the bound of seq_sum_f32, or, undecided, the sequential loop with each
// value taken from its lane by readlane. Unit (n_chunks, t) forms token t's
// gates per v head in place: beta_raw becomes beta = sigmoid(beta_raw),
// alpha becomes exp(gate), gate = softplus(alpha + dt_bias) * a
// (gdn_gates_kernel, then the step's exp of the gate).
constexpr int kConvUnits = 4;  // units (waves) per workgroup
__global__ __launch_bounds__(64 * kConvUnits) void gdn_conv_norm_rows_kernel(
    const float *__restrict__ win, const float *__restrict__ kern, const float *__restrict__ qkv,
    float *__restrict__ cv, int d_conv, int channels, int hd, int n_qk, float eps, float *__restrict__ beta,
    float *__restrict__ gexp, const float *__restrict__ dt_bias, const float *__restrict__ a, int n_v) {
    const int lane = threadIdx.x & 63, t = blockIdx.y, n_chunks = channels / hd;
    const int b = blockIdx.x * kConvUnits + (int)(threadIdx.x >> 6);
    if (b > n_chunks) return;  // the whole wave
    if (b == n_chunks) {
        for (int h = lane; h < n_v; h += 64) {
            const size_t i = (size_t)t * n_v + h;
            const float br = beta[i], al = gexp[i];
            beta[i] = sigmoid1(br);
            gexp[i] = expf_cr(__fmul_rn(softplus1(__fadd_rn(al, dt_bias[h])), a[h]));
        }
        return;
    }
    const bool norm = b < 2 * n_qk;  // wave-uniform
    float v[2] = {0.0f, 0.0f};
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int j = lane + 64 * k;
        if (j >= hd) break;
        const int c = b * hd + j;
        float x = 0.0f;
        for (int tau = 0; tau < d_conv; tau++) {
            const int u = t + tau;
            const float xv = u < d_conv - 1 ? win[(size_t)u * channels + c] : qkv[(size_t)(u - d_conv + 1) * channels + c];
            x = __fadd_rn(x, __fmul_rn(xv, kern[(size_t)c * d_conv + tau]));
        }
        v[k] = silu1(x);
        if (norm)
            s += (double)__fmul_rn(v[k], v[k]);
        else
            cv[(size_t)t * channels + c] = v[k];
    }
    if (!norm) return;
    // l2_norm_rows of the chunk: (float) of the sequential f64 sum of squares
    const double S = wave_sum_d(s);  // the same in every lane
    const double e = (double)(hd + 66) * 0x1p-52 * S;
    float sum32 = (float)(S - e);
    if (__float_as_uint(sum32) != __float_as_uint((float)(S + e))) {  // wave-uniform; -0 and +0 replay too
        double q = 0.0;
        for (int i = 0; i < hd; i++) {
            const float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(i < 64 ? v[0] : v[1]), i & 63));
            q += (double)__fmul_rn(x, x);
        }
        sum32 = (float)q;
    }
    const float scale = __fdiv_rn(1.0f, fmaxf(sqrtf_cr(sum32), eps));
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int j = lane + 64 * k;
        if (j < hd) cv[(size_t)t * channels + b * hd + j] = __fmul_rn(v[k], scale);
    }
}

// The conv window after nt steps, in place, one thread per channel: the
// sequence is the window's rows 0 .. d_conv - 2 followed by the nt qkv rows;
// rows 0 .. d_conv - 2 become its last d_conv - 1 entries and row d_conv - 1
// the last qkv row (as each step writes the token's qkv to the last row,
// then shifts rows 1 .. d_conv - 1 up). Row r's source is at index nt + r
// > r, so ascending r reads every old row before it is overwritten.
// Channel c of it; the workgroups of gdn_scan_kernel past the scan's own
// run it (the scan reads no window, and the conv before it is done with it).
__device__ __forceinline__ void conv_window_channel(float *__restrict__ win, const float *__restrict__ qkv, int nt,
                                                    int d_conv, int channels, int c) {
    for (int r = 0; r < d_conv - 1; r++) {
        const int u = nt + r;
        win[(size_t)r * channels + c] =
            u < d_conv - 1 ? win[(size_t)u * channels + c] : qkv[(size_t)(u - (d_conv - 1)) * channels + c];
    }
    win[(size_t)(d_conv - 1) * channels + c] = qkv[(size_t)(nt - 1) * channels + c];
}

// The delta rule (gdn_step_wg_kernel) of nt tokens, token after token, with
// no exchange between waves: lane l of wave w holds rows [R m, R m + R),
// m = l % RB (RB = dim / R lanes per column), of column j = (64 / RB)
// (kScanWaves blockIdx.x + w) + l / RB of v head blockIdx.y's state, in
// VGPRs for all the tokens. Each f64 dot is the lane's R terms, then a
// fixed tree over the column's RB lanes, with the bound of the step kernel: when
// both ends of [S - e, S + e] round to one f32 that is the reference's
// (float) of its sequential sum; otherwise the column's products go through
// the wave's LDS rows and every lane of the column sums them in the
// reference's order. Token t's q and k (normalised) and v are row t of cv,
// its beta and exp(gate) row t of beta / gexp; the next token's are loaded
// while this one is processed. out[t] receives o * scale (before the gated
// rmsnorm). The waves of a workgroup share nothing but are four to a
// workgroup so that they sit on the CU's four SIMDs: eight rows per lane
// (twice the waves of sixteen, half the instructions each) measured 294 us
// for 512 tokens of a 128-dim head as single-wave workgroups, which the
// hardware doubled up on SIMDs, as sixteen rows per lane did (288 us), and
// 226 us four to a workgroup.
constexpr int kScanWaves = 4;
template <int RB>
__device__ __forceinline__ double col_sum_d(double v) {
    v += dpp_d<0xB1>(v);
    v += dpp_d<0x4E>(v);
    if constexpr (RB >= 8) v += dpp_d<0x141>(v);
    if constexpr (RB == 16) v += dpp_d<0x140>(v);
    return v;
}
template <int RB, int R>
__global__ __launch_bounds__(64 * kScanWaves) void gdn_scan_kernel(const float *__restrict__ cv, const float *__restrict__ beta,
                                                      const float *__restrict__ gexp, float *__restrict__ state,
                                                      float *__restrict__ out, int nt, int channels, int n_qk,
                                                      int n_v, float scale, float *__restrict__ win,
                                                      const float *__restrict__ qkv, int d_conv) {
    if ((int)blockIdx.y >= n_v) {  // the window's workgroups, dispatched after the scan's (the whole workgroup)
        const int c = (((int)blockIdx.y - n_v) * (int)gridDim.x + (int)blockIdx.x) * 64 * kScanWaves + (int)threadIdx.x;
        if (c < channels) conv_window_channel(win, qkv, nt, d_conv, channels, c);
        return;
    }
    constexpr int dim = R * RB, CPW = 64 / RB;  // columns per wave
    __shared__ float prodw[kScanWaves][CPW][dim];  // per wave: a column's products, for the ordered replay
    const int wv = (int)(threadIdx.x >> 6);
    float (*prod)[dim] = prodw[wv];
    const int lane = threadIdx.x & 63, m = lane % RB, jc = lane / RB, h = blockIdx.y, hq = h % n_qk;
    const int j = (blockIdx.x * kScanWaves + wv) * CPW + jc, i0 = R * m;
    float *S = state + (size_t)h * dim * dim + (size_t)i0 * dim + j;
    float cs[R];
#pragma unroll
    for (int r = 0; r < R; r++) cs[r] = S[(size_t)r * dim];
    const size_t oq = (size_t)hq * dim + i0, ok = (size_t)(n_qk + hq) * dim + i0, ov = (size_t)(2 * n_qk + h) * dim + j;
    // inputs of two tokens (ping-pong: token t in buffer t & 1, so the
    // next token's loads land in registers no instruction of this token reads)
    float qn[2][R], kn[2][R], vn[2], gn[2], bn[2];
    auto fetch = [&](int t, int bsel) {
        const float4 *q4 = (const float4 *)(cv + (size_t)t * channels + oq);
        const float4 *k4 = (const float4 *)(cv + (size_t)t * channels + ok);
#pragma unroll
        for (int u = 0; u < R / 4; u++) {
            const float4 a = q4[u], b = k4[u];
            qn[bsel][4 * u] = a.x, qn[bsel][4 * u + 1] = a.y, qn[bsel][4 * u + 2] = a.z, qn[bsel][4 * u + 3] = a.w;
            kn[bsel][4 * u] = b.x, kn[bsel][4 * u + 1] = b.y, kn[bsel][4 * u + 2] = b.z, kn[bsel][4 * u + 3] = b.w;
        }
        vn[bsel] = cv[(size_t)t * channels + ov];
        gn[bsel] = gexp[(size_t)t * n_v + h];
        bn[bsel] = beta[(size_t)t * n_v + h];
    };
    // (float) of the reference's sequential f64 sum over i < dim of cs_i x_i
    auto dot = [&](const float *x) {
        // four interleaved partial sums (the bound covers any order), then
        // a fixed tree
        double s4[4] = {0.0, 0.0, 0.0, 0.0}, a4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int r = 0; r < R; r++) {
            const double t = (double)__fmul_rn(cs[r], x[r]);
            s4[r & 3] += t;
            a4[r & 3] += fabs(t);
        }
        const double s = (s4[0] + s4[1]) + (s4[2] + s4[3]), ab = (a4[0] + a4[1]) + (a4[2] + a4[3]);
        const double Sc = col_sum_d<RB>(s), Ac = col_sum_d<RB>(ab);
        const double e = (double)(dim + 66) * 0x1p-52 * Ac;
        const float lo = (float)(Sc - e), hi = (float)(Sc + e);
        const bool undecided = __float_as_uint(lo) != __float_as_uint(hi);
        if (!__builtin_amdgcn_ballot_w64(undecided)) return lo;
#pragma unroll
        for (int r = 0; r < R; r++) prod[jc][i0 + r] = __fmul_rn(cs[r], x[r]);
        // the rows are this wave's own: wave-scope ordering of the LDS
        // writes before the reads (a workgroup barrier would also wait for
        // the other waves and the next token's global loads)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float res = lo;
        if (undecided) {
            double q = 0.0;
            for (int i = 0; i < dim; i++) q += (double)prod[jc][i];
            res = (float)q;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        return res;
    };
    auto step = [&](int t, int bsel) {
        // unconditional (the last token fetches itself again): a fetch under
        // a branch makes the compiler's load counters assume the branch not
        // taken, and this token's reads then wait for the next token's loads
        fetch(min(t + 1, nt - 1), bsel ^ 1);
        const float *kc = kn[bsel], *qc = qn[bsel];
#pragma unroll
        for (int r = 0; r < R; r++) cs[r] = __fmul_rn(cs[r], gn[bsel]);
        const float sum = dot(kc);
        const float d = __fmul_rn(__fsub_rn(vn[bsel], sum), bn[bsel]);
#pragma unroll
        for (int r = 0; r < R; r++) cs[r] = __fadd_rn(cs[r], __fmul_rn(kc[r], d));
        const float o = dot(qc);
        // every lane of the column holds o: all store it (the same value to
        // the same address), with no branch around the store
        out[(size_t)t * n_v * dim + (size_t)h * dim + j] = __fmul_rn(o, scale);
    };
    fetch(0, 0);
    for (int t = 0; t < nt; t += 2) {
        step(t, 0);
        if (t + 1 < nt) step(t + 1, 1);
    }
#pragma unroll
    for (int r = 0; r < R; r++) S[(size_t)r * dim] = cs[r];
}

// The rope rotation (kernels.rs:121-123): f64 sin/cos, fma, rounded to f32.
__device__ __forceinline__ void rotate_pair(float *a, float *b, double angle) {
    double s, c;
    sincos(angle, &s, &c);
    const double x0 = (double)*a, x1 = (double)*b;
    *a = (float)fma(c, x0, -(s * x1));
    *b = (float)fma(s, x0, c * x1);
}

// mode 0: llama pairs (2i, 2i+1); 1: neox pairs (i, i + n/2); each over
// rows of n; one thread per pair.
__global__ void rope_freq_kernel(int mode, float *__restrict__ x, int rows, int n, const float *__restrict__ freqs,
                                 double pos) {
    const int half = n / 2;
    const size_t total = (size_t)rows * half;
    for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < total; t += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(t / half), i = (int)(t % half);
        float *xr = x + (size_t)r * n;
        const double angle = pos * (double)freqs[i];
        if (mode == 0)
            rotate_pair(&xr[2 * i], &xr[2 * i + 1], angle);
        else
            rotate_pair(&xr[i], &xr[i + half], angle);
    }
}

// rope_apply_imrope (kernels.rs:381-400): pair ic rotates when ic % 3 == 0
// by pos * theta^ic, the product formed by the reference's running
// multiplication (one f64 rounding per pair before it).
__global__ void rope_imrope_kernel(float *__restrict__ x, int rows, int n, int n_rot, double theta_scale, double pos) {
    const int half = n_rot / 2, nrot3 = (half + 2) / 3;
    const size_t total = (size_t)rows * nrot3;
    for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < total; t += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(t / nrot3), ic = 3 * (int)(t % nrot3);
        double angle = pos;
        for (int i = 0; i < ic; i++) angle *= theta_scale;
        float *xr = x + (size_t)r * n;
        rotate_pair(&xr[ic], &xr[ic + half], angle);
    }
}

// The pairwise tree (kernels.rs:27-42) of len <= 64 values held one per
// lane, level by level: lane i forms node i from lanes 2i and 2i+1, an odd
// tail carried up. Returned to every lane.
__device__ double wave_tree(double v, int len) {
    const int lane = threadIdx.x & 63;
    while (len > 1) {
        const double a = __shfl(v, (2 * lane) & 63), b = __shfl(v, (2 * lane + 1) & 63);
        v = 2 * lane + 1 < len ? a + b : a;
        len = (len + 1) >> 1;
    }
    return __shfl(v, 0);
}

// The pairwise tree of leaf(0), ..., leaf(n - 1), n <= 64^3, by one wave.
// Chunks of 64 and of 4096 (powers of two) are nodes of the tree, with the
// remainder's own tree as the carried last node, so the tree is the tree
// over the chunk sums, level after level.
constexpr int kWaveTreeMax = 64 * 64 * 64;
template <class Leaf>
__device__ double wave_pairwise_n(Leaf leaf, int n) {
    const int lane = threadIdx.x & 63;
    double l2 = 0.0;
    int m2 = 0;
    for (int b2 = 0; b2 < n; b2 += 4096, m2++) {
        const int n2 = min(4096, n - b2);
        double l1 = 0.0;
        int m1 = 0;
        for (int b1 = 0; b1 < n2; b1 += 64, m1++) {
            const int c = min(64, n2 - b1);
            const double s = wave_tree(lane < c ? leaf(b2 + b1 + lane) : 0.0, c);
            if (lane == m1) l1 = s;
        }
        const double s2 = wave_tree(l1, m1);
        if (lane == m2) l2 = s2;
    }
    return wave_tree(l2, m2);
}

// matmul_f32_acc (kernels.rs:87-101): one wave per output element, products
// a*b exact in f64, pairwise sum over k, acc + sum in f64, rounded once.
__global__ __launch_bounds__(OPS_TPB) void matmul_acc_kernel(float *__restrict__ acc, const float *__restrict__ a,
                                                             const float *__restrict__ b, int m, int k, int n) {
    const size_t o = (size_t)blockIdx.x * (OPS_TPB / 64) + (threadIdx.x >> 6);
    if (o >= (size_t)m * n) return;  // whole waves
    const int i = (int)(o / n), j = (int)(o % n);
    const float *ar = a + (size_t)i * k;
    const double s = wave_pairwise_n([&](int l) { return (double)ar[l] * (double)b[(size_t)l * n + j]; }, k);
    if ((threadIdx.x & 63) == 0) acc[o] = (float)((double)acc[o] + s);
}

// ---- decode attention (qwen35_forward.rs:639-671) ----
// Caches are [n_ctx][n_head_kv][hd] f32; q head h reads kv head h / group
// (group = n_head / n_head_kv, consecutive heads share a kv head).

// Pairwise sum (kernels.rs:21-42) of 64 * E values, lane l holding values
// [E*l, E*l + E). For a power-of-two count the tree adds adjacent nodes
// level by level: the lane-local tree, then the xor butterfly over lanes
// (both lanes of a pair form the same node: f64 addition is commutative).
template <int E>
__device__ double wave_pairwise(double (&t)[E]) {
#pragma unroll
    for (int w = E; w > 1; w /= 2)
#pragma unroll
        for (int j = 0; j < w / 2; j++) t[j] = t[2 * j] + t[2 * j + 1];
    double s = t[0];
#pragma unroll
    for (int off = 1; off < 64; off *= 2) s = s + __shfl_xor(s, off);
    return s;
}

constexpr int kAttnMaxGroup = 8;
constexpr int kScoresPPB = 8;  // positions per workgroup (2 per wave)

// scores[h][p] = (f32) dot_f32(q_h, K[p][kv]) for the group's heads; one
// wave per position, E = hd / 64 values per lane. Query z = blockIdx.z (of
// a prefill) sees n_ctx + z positions; its q and scores are z q_st and
// z sc_st floats on.
template <int E>
__global__ __launch_bounds__(OPS_TPB) void attn_scores_kernel(float *__restrict__ scores, const float *__restrict__ q,
                                                              const float *__restrict__ kc, int n_ctx, int n_head_kv,
                                                              int group, size_t q_st, size_t sc_st) {
    constexpr int HD = 64 * E;
    __shared__ float qs[kAttnMaxGroup * HD];
    n_ctx += (int)blockIdx.z;
    if (blockIdx.x * kScoresPPB >= (unsigned)n_ctx) return;  // the whole workgroup: past this query's positions
    q += blockIdx.z * q_st;
    scores += blockIdx.z * sc_st;
    const int kv = blockIdx.y, lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    for (int t = threadIdx.x; t < group * HD; t += OPS_TPB) qs[t] = q[(size_t)kv * group * HD + t];
    __syncthreads();
    const size_t kv_len = (size_t)n_head_kv * HD;
    // the wave's positions p0 + 4t: every K row is loaded before the dots
    constexpr int PW = kScoresPPB / (OPS_TPB / 64);
    const int p0 = blockIdx.x * kScoresPPB + w;
    float kx[PW][E];
#pragma unroll
    for (int t = 0; t < PW; t++) {
        const int p = min(p0 + t * (OPS_TPB / 64), n_ctx - 1);
        const float *kr = kc + (size_t)p * kv_len + (size_t)kv * HD + lane * E;
#pragma unroll
        for (int e = 0; e < E; e++) kx[t][e] = kr[e];
    }
#pragma unroll
    for (int t = 0; t < PW; t++) {
        const int p = p0 + t * (OPS_TPB / 64);
        if (p >= n_ctx) break;  // wave-uniform
        for (int g = 0; g < group; g++) {
            double d[E];
#pragma unroll
            for (int e = 0; e < E; e++) d[e] = (double)qs[g * HD + lane * E + e] * (double)kx[t][e];
            const double sc = wave_pairwise<E>(d);
            if (lane == 0) scores[(size_t)(kv * group + g) * n_ctx + p] = (float)sc;
        }
    }
}

// The pairwise tree (kernels.rs:21-42) of the N products x_i * y_i (exact
// in f64), i in [B, B + N), N a power of two: both halves, then their sum,
// the reference's adjacent-pair levels (it carries no odd tail at a power
// of two). x a broadcast row in LDS, y the lane's row in LDS.
template <int N, int B>
__device__ __forceinline__ double tree_dot(const float *__restrict__ x, const float *__restrict__ y) {
    if constexpr (N == 1)
        return (double)x[B] * (double)y[B];
    else if constexpr (N == 2)  // x1 y1 + x0 y0, both exact, rounded once: one fma
        return fma((double)x[B + 1], (double)y[B + 1], (double)x[B] * (double)y[B]);
    else
        return tree_dot<N / 2, B>(x, y) + tree_dot<N / 2, B + N / 2>(x, y);
}

// Scores of a prefill chunk with one lane per position: the workgroup holds
// the K rows of 64 positions (one kv head) in LDS and the q rows of up to qb
// queries of the group's heads (at most 80 KB in all, so two workgroups
// share a CU); wave w takes the (query, head)
// pairs w, w + 4, ..., and each lane forms its position's whole dot as the
// pairwise tree, with no exchange between lanes. Query z0 + zz sees n_ctx +
// z0 + zz positions (causal). Each dot is the same tree of the same exact
// products as attn_scores_kernel's, so the same bits; the lane butterflies
// that bound that kernel are gone.
constexpr int kLaneScoresPos = 64;
template <int HD>
__global__ __launch_bounds__(OPS_TPB) void attn_scores_lane_kernel(float *__restrict__ scores,
                                                                   const float *__restrict__ q,
                                                                   const float *__restrict__ kc, int n_ctx,
                                                                   int n_head_kv, int group, size_t q_st,
                                                                   size_t sc_st, int rows, int qb) {
    constexpr int KP = HD + 1;  // K row pitch in floats: an odd pitch, no bank conflicts
    extern __shared__ __align__(16) float qd[];  // [qb * group][HD], then K [64][KP]
    const int p0 = blockIdx.x * kLaneScoresPos, kv = blockIdx.y, z0 = blockIdx.z * qb;
    const int nz = min(qb, rows - z0), n_hi = n_ctx + z0 + nz - 1;  // positions of the block's last query
    if (p0 >= n_hi) return;  // the whole workgroup
    float *ks = qd + (size_t)qb * group * HD;
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gh = group * HD;
    const size_t kv_len = (size_t)n_head_kv * HD;
    for (int idx = tid; idx < kLaneScoresPos * (HD / 4); idx += OPS_TPB) {
        const int r = idx / (HD / 4), c4 = idx - r * (HD / 4);
        const int p = min(p0 + r, n_hi - 1);
        const float4 v = *(const float4 *)(kc + (size_t)p * kv_len + (size_t)kv * HD + 4 * c4);
        float *d = ks + r * KP + 4 * c4;
        d[0] = v.x, d[1] = v.y, d[2] = v.z, d[3] = v.w;
    }
    for (int idx = tid; idx < nz * gh; idx += OPS_TPB) {
        const int zz = idx / gh, rr = idx - zz * gh;
        qd[idx] = q[(size_t)(z0 + zz) * q_st + (size_t)kv * gh + rr];
    }
    __syncthreads();
    const int p = p0 + lane;
    const float *kr = ks + lane * KP;
    for (int pair = wv; pair < nz * group; pair += OPS_TPB / 64) {
        const int zz = pair / group, g = pair - zz * group;
        const int nzc = n_ctx + z0 + zz;
        if (p0 >= nzc) continue;  // no position of the tile for this query (wave-uniform)
        const double sc = tree_dot<HD, 0>(qd + (size_t)pair * HD, kr);
        if (p < nzc) scores[(size_t)(z0 + zz) * sc_st + (size_t)(kv * group + g) * nzc + p] = (float)sc;
    }
}

// out[h][i] = (f32) of the sequential f64 sum over p of soft[h][p] * V[p][i]
// (every product exact in f64). Lane = column i, the waves split p; the
// partial sums S and absolute sums A meet in LDS. Any summation order of
// n terms lies within gamma_n * A of the exact sum, so the sequential sum
// lies in [S - e, S + e], e = (n + 66) 2^-52 A (with room for the rounding
// of e and S +- e); when both ends round to the same f32 (same bits) that
// is the reference's value, else the lane replays the sequential loop.
constexpr int kPvBatch = 16;  // positions whose V loads a wave issues before summing
constexpr int kPvCoop = 4;    // at most this many replays per wave run one column at a time
constexpr int kPvChunk = 8;   // positions per lane loaded at once in such a replay
template <int G>
constexpr int pv_waves() { return G <= 4 ? 16 : 8; }  // the LDS partials stay within 64 KB
// G: q heads per kv head, compile-time so that a batch's loads issue back to
// back. Query z = blockIdx.z (of a prefill) sees n_ctx + z positions; its
// soft, out, gz and gated rows are z times the strides in st on.
struct PvStrides {
    size_t soft, out, gz, gated;
};
template <int G>
__global__ __launch_bounds__(pv_waves<G>() * 64) void attn_pv_kernel(float *__restrict__ out,
                                                                    const float *__restrict__ soft,
                                                                    const float *__restrict__ vc, int n_ctx,
                                                                    int n_head_kv, int hd,
                                                                    const float *__restrict__ gz, int gzs,
                                                                    float *__restrict__ gated, PvStrides zs) {
    constexpr int group = G, kPvWaves = pv_waves<G>();
    __shared__ double part[2][kPvWaves][G][64];
    n_ctx += (int)blockIdx.z;
    soft += blockIdx.z * zs.soft;
    out += blockIdx.z * zs.out;
    if (gated) {
        gz += blockIdx.z * zs.gz;
        gated += blockIdx.z * zs.gated;
    }
    const int kv = blockIdx.y, lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i = blockIdx.x * 64 + lane;
    const size_t kv_len = (size_t)n_head_kv * hd;
    const float *vcol = vc + (size_t)kv * hd + i;
    const float *sr = soft + (size_t)kv * group * n_ctx;
    double S[G], A[G];
#pragma unroll
    for (int g = 0; g < G; g++) S[g] = A[g] = 0.0;
    // positions in batches of kPvBatch per wave, loads first (the sums only
    // need some order: the bound below covers any)
    for (int p0 = w; p0 < n_ctx; p0 += kPvWaves * kPvBatch) {
        float vb[kPvBatch], sb[kPvBatch][G];
#pragma unroll
        for (int u = 0; u < kPvBatch; u++) {
            const int p = min(p0 + u * kPvWaves, n_ctx - 1);
            vb[u] = vcol[(size_t)p * kv_len];
#pragma unroll
            for (int g = 0; g < G; g++) sb[u][g] = sr[(size_t)g * n_ctx + p];
        }
#pragma unroll
        for (int u = 0; u < kPvBatch; u++) {
            const bool in = p0 + u * kPvWaves < n_ctx;
#pragma unroll
            for (int g = 0; g < G; g++) {
                const double t = in ? (double)sb[u][g] * (double)vb[u] : 0.0;
                S[g] += t;
                A[g] += fabs(t);
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
        part[0][w][g][lane] = S[g];
        part[1][w][g][lane] = A[g];
    }
    __syncthreads();
    double st = 0.0, at = 0.0;
    if (w < group)
        for (int u = 0; u < kPvWaves; u++) {
            st += part[0][u][w][lane];
            at += part[1][u][w][lane];
        }
    __syncthreads();  // part is free: a replay below uses it as its wave's scratch
    if (w < group) {
        const int g = w;
        const double e = (double)(n_ctx + 66) * 0x1p-52 * at;
        const float lo = (float)(st - e), hi = (float)(st + e);
        float r = lo;
        // the reference's sequential sum where the bound cannot decide
        // (about 1e-4 of the outputs)
        const bool need = __float_as_uint(lo) != __float_as_uint(hi);
        unsigned long long mask = __ballot(need);
        if (__popcll(mask) > kPvCoop) {
            // many columns: each lane replays its own, loads in batches, the adds in order
            if (need) {
                constexpr int RB = 32;
                double q = 0.0;
                for (int p0 = 0; p0 < n_ctx; p0 += RB) {
                    float vb[RB], sb[RB];
#pragma unroll
                    for (int u = 0; u < RB; u++) {
                        const int p = min(p0 + u, n_ctx - 1);
                        vb[u] = vcol[(size_t)p * kv_len];
                        sb[u] = sr[(size_t)g * n_ctx + p];
                    }
#pragma unroll
                    for (int u = 0; u < RB; u++)
                        if (p0 + u < n_ctx) q += (double)sb[u] * (double)vb[u];
                }
                r = (float)q;
            }
        } else {
            // a few columns: the wave replays them one at a time, every lane
            // forming the products of its positions (loads in parallel) into
            // the wave's LDS scratch, then all lanes adding them in position
            // order (broadcast reads; the same sum in each lane)
            double *buf = &part[0][0][0][0] + (size_t)w * 64 * kPvChunk;  // within part: kPvWaves >= 4
            while (mask) {
                const int l = __ffsll(mask) - 1;
                mask &= mask - 1;
                const float *vl = vc + (size_t)kv * hd + blockIdx.x * 64 + l;
                double q = 0.0;
                for (int p0 = 0; p0 < n_ctx; p0 += 64 * kPvChunk) {
#pragma unroll
                    for (int k = 0; k < kPvChunk; k++) {
                        const int p = min(p0 + 64 * k + lane, n_ctx - 1);
                        buf[64 * k + lane] = (double)sr[(size_t)g * n_ctx + p] * (double)vl[(size_t)p * kv_len];
                    }
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    const int m = min(64 * kPvChunk, n_ctx - p0);
                    // the reads of the next 8 values issue before the adds of these 8
                    int p = 0;
                    double b[8];
                    if (m >= 8) {
#pragma unroll
                        for (int u = 0; u < 8; u++) b[u] = buf[u];
                    }
                    for (; p + 8 <= m; p += 8) {
                        double nb[8];
                        const int pn = p + 16 <= m ? p + 8 : p;  // the last batch rereads itself
#pragma unroll
                        for (int u = 0; u < 8; u++) nb[u] = buf[pn + u];
#pragma unroll
                        for (int u = 0; u < 8; u++) q += b[u];
#pragma unroll
                        for (int u = 0; u < 8; u++) b[u] = nb[u];
                    }
                    for (; p < m; p++) q += buf[p];
                    // every lane's reads are done before the next chunk's writes
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                }
                if (lane == l) r = (float)q;
            }
        }
        out[(size_t)(kv * group + g) * hd + i] = r;
        // the gated output (qwen35_forward.rs:677-684, as mul_act_kernel)
        if (gated) gated[(size_t)(kv * group + g) * hd + i] = __fmul_rn(r, sigmoid1(gz[(size_t)(kv * group + g) * gzs + i]));
    }
}

// attn_pv_kernel for a prefill chunk: a workgroup takes the NP = (16 / G) *
// G (query, head) pairs of QB = 16 / G consecutive queries and the G heads
// of kv head blockIdx.y, lane = column blockIdx.x * 64 + lane, so each V
// load serves all NP pairs. Wave w takes the 16-position batches w, w + 4,
// ...; a pair's soft values of a batch are uniform (scalar) loads. Each
// product is exact in f64, so S += s * v and A += |s * v| are single fused
// multiply-adds with the values of the separate multiply and add. The four
// waves' S and A meet in LDS, then the bound decides each output as in
// attn_pv_kernel, or the lane replays the sequential sum.
constexpr int kPvRowsWaves = 4, kPvRowsBatch = 16;
template <int G>
__global__ __launch_bounds__(kPvRowsWaves * 64) void attn_pv_rows_kernel(
    float *__restrict__ out, const float *__restrict__ soft, const float *__restrict__ vc, int n_ctx, int n_head_kv,
    int hd, int rows, const float *__restrict__ gz, int gzs, float *__restrict__ gated, PvStrides zs) {
    constexpr int QB = 16 / G, NP = QB * G;
    __shared__ double part[kPvRowsWaves][NP][64];
    static_assert(NP >= kPvChunk, "a wave's part rows hold its replay chunk");
    const int kv = blockIdx.y, lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int z0 = blockIdx.z * QB, nz = min(QB, rows - z0);
    const int i = blockIdx.x * 64 + lane;
    const size_t kv_len = (size_t)n_head_kv * hd;
    const float *vcol = vc + (size_t)kv * hd + i;
    const int n_hi = n_ctx + z0 + nz - 1;  // positions of the block's last query
    // soft row of pair q: query z0 + q / G, head kv * G + q % G
    auto srow = [&](int q) {
        const int zz = q / G, nzc = n_ctx + z0 + zz;
        return soft + (size_t)(z0 + zz) * zs.soft + (size_t)(kv * G + q % G) * nzc;
    };
    double S[NP], A[NP];
#pragma unroll
    for (int q = 0; q < NP; q++) S[q] = A[q] = 0.0;
    for (int pb = w * kPvRowsBatch; pb < n_hi; pb += kPvRowsWaves * kPvRowsBatch) {
        double vd[kPvRowsBatch];
#pragma unroll
        for (int u = 0; u < kPvRowsBatch; u++) vd[u] = (double)vcol[(size_t)min(pb + u, n_hi - 1) * kv_len];
#pragma unroll
        for (int q = 0; q < NP; q++) {
            const int zz = q / G, nzc = n_ctx + z0 + zz;
            if (zz >= nz || pb >= nzc) continue;  // wave-uniform
            const float *sr = srow(q) + pb;
            if (pb + kPvRowsBatch <= nzc) {
#pragma unroll
                for (int u = 0; u < kPvRowsBatch; u++) {
                    const double sv = (double)sr[u];
                    S[q] = fma(sv, vd[u], S[q]);
                    A[q] = fma(fabs(sv), fabs(vd[u]), A[q]);
                }
            } else {
                const int m = nzc - pb;
#pragma unroll
                for (int u = 0; u < kPvRowsBatch; u++)
                    if (u < m) {
                        const double sv = (double)sr[u];
                        S[q] = fma(sv, vd[u], S[q]);
                        A[q] = fma(fabs(sv), fabs(vd[u]), A[q]);
                    }
            }
        }
    }
    // the waves' partials: S, then A, through the one LDS array
    double st[(NP + kPvRowsWaves - 1) / kPvRowsWaves], at[(NP + kPvRowsWaves - 1) / kPvRowsWaves];
#pragma unroll
    for (int ph = 0; ph < 2; ph++) {
#pragma unroll
        for (int q = 0; q < NP; q++) part[w][q][lane] = ph == 0 ? S[q] : A[q];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < (NP + kPvRowsWaves - 1) / kPvRowsWaves; k++) {
            const int q = w + kPvRowsWaves * k;
            double t = 0.0;
            if (q < NP)
#pragma unroll
                for (int u = 0; u < kPvRowsWaves; u++) t += part[u][q][lane];
            (ph == 0 ? st : at)[k] = t;
        }
        __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < (NP + kPvRowsWaves - 1) / kPvRowsWaves; k++) {
        const int q = w + kPvRowsWaves * k;
        if (q >= NP) break;
        const int zz = q / G, g = q % G, nzc = n_ctx + z0 + zz;
        if (zz >= nz) break;  // wave-uniform; later k only higher zz
        const double e = (double)(nzc + 66) * 0x1p-52 * at[k];
        const float lo = (float)(st[k] - e), hi = (float)(st[k] + e);
        float r = lo;
        // the reference's sequential sum where the bound cannot decide
        const bool need = __float_as_uint(lo) != __float_as_uint(hi);
        unsigned long long mask = __ballot(need);
        const float *sr = srow(q);
        if (__popcll(mask) > kPvCoop) {
            // many columns: each lane replays its own
            if (need) {
                double qs = 0.0;
                for (int p0 = 0; p0 < nzc; p0 += 16) {
                    float vb[16], sb[16];
#pragma unroll
                    for (int u = 0; u < 16; u++) {
                        const int p = min(p0 + u, nzc - 1);
                        vb[u] = vcol[(size_t)p * kv_len];
                        sb[u] = sr[p];
                    }
#pragma unroll
                    for (int u = 0; u < 16; u++)
                        if (p0 + u < nzc) qs += (double)sb[u] * (double)vb[u];
                }
                r = (float)qs;
            }
        } else {
            // a few columns, one at a time: every lane forms the products of
            // its positions (loads in parallel) into the wave's LDS scratch
            // (part is free after the reductions), then all lanes add them in
            // position order (broadcast reads; the same sum in each lane)
            double *buf = &part[w][0][0];
            while (mask) {
                const int l = __ffsll(mask) - 1;
                mask &= mask - 1;
                const float *vl = vc + (size_t)kv * hd + blockIdx.x * 64 + l;
                double qs = 0.0;
                for (int p0 = 0; p0 < nzc; p0 += 64 * kPvChunk) {
#pragma unroll
                    for (int c = 0; c < kPvChunk; c++) {
                        const int p = min(p0 + 64 * c + lane, nzc - 1);
                        buf[64 * c + lane] = (double)sr[p] * (double)vl[(size_t)p * kv_len];
                    }
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    const int m = min(64 * kPvChunk, nzc - p0);
                    // the reads of the next eight values issue before the adds of these eight
                    int p = 0;
                    double bb[8];
                    if (m >= 8) {
#pragma unroll
                        for (int u = 0; u < 8; u++) bb[u] = buf[u];
                    }
                    for (; p + 8 <= m; p += 8) {
                        double nb[8];
                        const int pn = p + 16 <= m ? p + 8 : p;  // the last group rereads itself
#pragma unroll
                        for (int u = 0; u < 8; u++) nb[u] = buf[pn + u];
#pragma unroll
                        for (int u = 0; u < 8; u++) qs += bb[u];
#pragma unroll
                        for (int u = 0; u < 8; u++) bb[u] = nb[u];
                    }
                    for (; p < m; p++) qs += buf[p];
                    // every lane's reads are done before the next chunk's writes
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                }
                if (lane == l) r = (float)qs;
            }
        }
        float *o = out + (size_t)(z0 + zz) * zs.out;
        o[(size_t)(kv * G + g) * hd + i] = r;
        if (gated)
            gated[(size_t)(z0 + zz) * zs.gated + (size_t)(kv * G + g) * hd + i] =
                __fmul_rn(r, sigmoid1(gz[(size_t)(z0 + zz) * zs.gz + (size_t)(kv * G + g) * gzs + i]));
    }
}

// ---- glue of the layer forward (qwen35_forward.rs:333-710) ----------------
// GatedDeltaNet gates (:405-419): beta = sigmoid(beta_raw), sp =
// softplus(alpha + dt_bias), gate = sp * a, per v head.
__global__ void gdn_gates_kernel(const float *__restrict__ beta_raw, const float *__restrict__ alpha,
                                 const float *__restrict__ dt_bias, const float *__restrict__ a,
                                 float *__restrict__ beta, float *__restrict__ sp, float *__restrict__ gate, int n) {
    for (int h = blockIdx.x * blockDim.x + threadIdx.x; h < n; h += gridDim.x * blockDim.x) {
        beta[h] = sigmoid1(beta_raw[h]);
        const float p = softplus1(__fadd_rn(alpha[h], dt_bias[h]));
        sp[h] = p;
        gate[h] = __fmul_rn(p, a[h]);
    }
}

// out[i] = y[i] * act(z[(i / n) * zs + i % n]), act 0 sigmoid (:679-683),
// 1 silu (:507-511): the activation is rounded to f32 first, as the
// reference's separate buffer.
__global__ void mul_act_kernel(int op, float *out, const float *y, const float *__restrict__ z, int n, int zs,
                               size_t total) {  // out may be y
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const float zv = z[(i / n) * zs + i % n];
        out[i] = __fmul_rn(y[i], op == 0 ? sigmoid1(zv) : silu1(zv));
    }
}

// out = a + b (the residual additions, :525-527, :534-536)
__global__ void add_kernel(float *__restrict__ out, const float *__restrict__ a, const float *__restrict__ b,
                           size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = __fadd_rn(a[i], b[i]);
}

// One launch for the GatedDeltaNet steps between the projections and the
// delta rule (qwen35_forward.rs:405-464): workgroup b < n_chunks runs the
// conv step (as conv_step_kernel) over channels [b*hd, (b+1)*hd), and for
// the q and k chunks (b < 2*n_qk) the l2 norm of the chunk (as l2norm_kernel,
// the chunk's values kept in LDS); the last workgroup forms the gates (as
// gdn_gates_kernel). Same operations in the same order as the three
// kernels, so the same bits.
constexpr int kConvNormMaxHd = 1024;
__global__ __launch_bounds__(OPS_TPB) void gdn_conv_norm_kernel(
    float *__restrict__ win, const float *__restrict__ kern, float *__restrict__ raw, float *__restrict__ act,
    int d_conv, int channels, int hd, int n_qk, float eps, const float *__restrict__ beta_raw,
    const float *__restrict__ alpha, const float *__restrict__ dt_bias, const float *__restrict__ a,
    float *__restrict__ beta, float *__restrict__ sp, float *__restrict__ gate, int n_v) {
    __shared__ float vals[kConvNormMaxHd];
    __shared__ double red[OPS_TPB / 64];
    __shared__ float bc;
    const int b = blockIdx.x, n_chunks = channels / hd;
    if (b == n_chunks) {
        for (int h = threadIdx.x; h < n_v; h += OPS_TPB) {
            beta[h] = sigmoid1(beta_raw[h]);
            const float p = softplus1(__fadd_rn(alpha[h], dt_bias[h]));
            sp[h] = p;
            gate[h] = __fmul_rn(p, a[h]);
        }
        return;
    }
    const bool norm = b < 2 * n_qk;  // workgroup-uniform
    double s = 0.0;
    for (int j = threadIdx.x; j < hd; j += OPS_TPB) {
        const int c = b * hd + j;
        float x[9];
        for (int r = 0; r < d_conv; r++) x[r] = win[(size_t)r * channels + c];
        float t = 0.0f;
        for (int tau = 0; tau < d_conv; tau++) t = __fadd_rn(t, __fmul_rn(x[tau], kern[(size_t)c * d_conv + tau]));
        raw[c] = t;
        const float v = silu1(t);
        for (int r = 1; r < d_conv; r++) win[(size_t)(r - 1) * channels + c] = x[r];
        if (norm) {
            vals[j] = v;
            s += (double)__fmul_rn(v, v);
        } else {
            act[c] = v;
        }
    }
    if (!norm) return;
    const double S = block_sum_d<OPS_TPB>(s, red);  // its barrier also publishes vals
    const float sum32 = seq_sum_f32<OPS_TPB>([](int i) { return vals[i]; }, hd, S, [](double v) { return (float)v; },
                                             &bc);
    const float scale = __fdiv_rn(1.0f, fmaxf(sqrtf_cr(sum32), eps));
    for (int j = threadIdx.x; j < hd; j += OPS_TPB) act[b * hd + j] = __fmul_rn(vals[j], scale);
}

// One launch for the attention layer's q and k preparation
// (qwen35_forward.rs:585-642): workgroup h < n_head normalises the first
// half of q head h (rmsnorm with attn_q_norm, as rmsnorm_kernel) into q_out
// row h, workgroup n_head + j the raw k row of kv head j (attn_k_norm) into
// k_out row j; then IMROPE rotates the row (as rope_imrope_kernel) before
// it is stored. Token z = blockIdx.y (of a prefill) is at position pos + z,
// its rows st[0..3] floats (qfull, q_out, k_raw, k_out) times z on.
constexpr int kQkMaxHd = 512;
struct QkStrides {
    size_t qfull, q_out, k_raw, k_out;
};
__global__ __launch_bounds__(OPS_TPB) void attn_qk_prep_kernel(const float *__restrict__ qfull, float *__restrict__ q_out,
                                                             const float *__restrict__ k_raw, float *__restrict__ k_out,
                                                             const float *__restrict__ wq, const float *__restrict__ wk,
                                                             int hd, int n_head, int n_rot, double theta_scale,
                                                             double pos, float eps, QkStrides st) {
    __shared__ float rowv[kQkMaxHd];
    __shared__ double red[OPS_TPB / 64];
    __shared__ float bc;
    const int b = blockIdx.x;
    qfull += blockIdx.y * st.qfull;
    q_out += blockIdx.y * st.q_out;
    k_raw += blockIdx.y * st.k_raw;
    k_out += blockIdx.y * st.k_out;
    pos += (double)blockIdx.y;
    const bool isq = b < n_head;
    const float *xr = isq ? qfull + (size_t)b * 2 * hd : k_raw + (size_t)(b - n_head) * hd;
    const float *w = isq ? wq : wk;
    float *yr = isq ? q_out + (size_t)b * hd : k_out + (size_t)(b - n_head) * hd;
    double s = 0.0;
    float wr[kQkMaxHd / OPS_TPB];  // the weights, loaded with x
#pragma unroll
    for (int k = 0; k < kQkMaxHd / OPS_TPB; k++) {
        const int i = threadIdx.x + k * OPS_TPB;
        wr[k] = i < hd ? w[i] : 0.0f;
    }
    for (int i = threadIdx.x; i < hd; i += OPS_TPB) {
        const float v = xr[i];
        rowv[i] = v;
        s += (double)__fmul_rn(v, v);
    }
    const double S = block_sum_d<OPS_TPB>(s, red);  // its barrier also publishes rowv
    const double dn = (double)hd;
    const float mean = seq_sum_f32<OPS_TPB>([](int i) { return rowv[i]; }, hd, S,
                                            [dn](double u) { return (float)(u / dn); }, &bc);
    const float scale = __fdiv_rn(1.0f, sqrtf_cr(__fadd_rn(mean, eps)));
#pragma unroll
    for (int k = 0; k < kQkMaxHd / OPS_TPB; k++) {
        const int i = threadIdx.x + k * OPS_TPB;
        if (i < hd) rowv[i] = __fmul_rn(__fmul_rn(rowv[i], scale), wr[k]);
    }
    __syncthreads();
    const int half = n_rot / 2, nrot3 = (half + 2) / 3;
    for (int t = threadIdx.x; t < nrot3; t += OPS_TPB) {
        const int ic = 3 * t;
        double angle = pos;
        for (int i = 0; i < ic; i++) angle *= theta_scale;
        rotate_pair(&rowv[ic], &rowv[ic + half], angle);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < hd; i += OPS_TPB) yr[i] = rowv[i];
}

inline unsigned ops_grid(size_t n) {
    const size_t g = (n + OPS_TPB - 1) / OPS_TPB;
    return (unsigned)(g < 65535u * 32u ? (g ? g : 1) : 65535u * 32u);
}

}  // namespace

hipError_t launch_rmsnorm(float *out, const float *x, const float *w, int n, int rows, float eps, hipStream_t s) {
    return launch_rmsnorm_rows(out, n, x, n, w, n, rows, eps, s);
}

hipError_t launch_rmsnorm_rows(float *out, int ys, const float *x, int xs, const float *w, int n, int rows, float eps,
                               hipStream_t s, const float *xb, float *xsum, const float *z, const Q8Planes *q8,
                               bool q6) {
    if (rows == 0 || n == 0) return hipSuccess;
    if (q8) {  // rows quantized into the q8k GEMM's planes in the same launch
        if (!rmsnorm_q8k_fits(n, rows) || q8->Mp < rows) return hipErrorInvalidValue;
        hipLaunchKernelGGL((rmsnorm_kernel<4, 1024, true>), dim3(q8->Mp), dim3(1024), 0, s, out, x, w, n, eps, xs, ys,
                           xb, xsum, z, *q8, rows, q6);
        return hipGetLastError();
    }
    if (n <= OPS_TPB)
        hipLaunchKernelGGL(rmsnorm_kernel<1>, dim3(rows), dim3(OPS_TPB), 0, s, out, x, w, n, eps, xs, ys, xb, xsum, z);
    else if (n <= 4 * 1024)  // wider rows: 1024 threads, four elements each
        hipLaunchKernelGGL((rmsnorm_kernel<4, 1024>), dim3(rows), dim3(1024), 0, s, out, x, w, n, eps, xs, ys, xb, xsum,
                           z);
    else if (n <= 16 * OPS_TPB)
        hipLaunchKernelGGL(rmsnorm_kernel<16>, dim3(rows), dim3(OPS_TPB), 0, s, out, x, w, n, eps, xs, ys, xb, xsum, z);
    else
        hipLaunchKernelGGL(rmsnorm_kernel<0>, dim3(rows), dim3(OPS_TPB), 0, s, out, x, w, n, eps, xs, ys, xb, xsum, z);
    return hipGetLastError();
}

hipError_t launch_l2norm(float *data, int dim, int rows, float eps, hipStream_t s) {
    if (rows == 0 || dim == 0) return hipSuccess;
    hipLaunchKernelGGL(l2norm_kernel, dim3(rows), dim3(OPS_TPB), 0, s, data, dim, eps);
    return hipGetLastError();
}

int softmax_max_len() { return kSmChunk * kSmMaxChunks; }

hipError_t launch_softmax(float *out, const float *x, int n, int rows, float scale, hipStream_t s) {
    if (rows == 0 || n == 0) return hipSuccess;
    if (n > softmax_max_len()) return hipErrorInvalidValue;
    if (n <= kSmWaveMax)
        hipLaunchKernelGGL(softmax_wave_kernel, dim3((rows + OPS_TPB / 64 - 1) / (OPS_TPB / 64)), dim3(OPS_TPB), 0, s,
                           out, x, n, scale, 0, (size_t)0, rows);
    else
        hipLaunchKernelGGL(softmax_kernel, dim3(rows), dim3(OPS_TPB), 0, s, out, x, n, scale, 0, (size_t)0);
    return hipGetLastError();
}

hipError_t launch_unary(int op, const float *x, size_t n, float *out, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(unary_kernel, dim3(ops_grid(n)), dim3(OPS_TPB), 0, s, op, x, n, out);
    return hipGetLastError();
}

hipError_t launch_ssm_conv(float *out, const float *x, const float *kern, int d_conv, int channels, int n_t,
                           hipStream_t s) {
    if (n_t == 0 || channels == 0) return hipSuccess;
    hipLaunchKernelGGL(ssm_conv_kernel, dim3(ops_grid((size_t)n_t * channels)), dim3(OPS_TPB), 0, s, out, x, kern,
                       d_conv, channels, n_t);
    return hipGetLastError();
}

hipError_t launch_gdn_step(float *state, float *out, const float *q, const float *k, const float *v, const float *gate,
                           const float *beta, int dim, int heads, float scale, hipStream_t s, int n_qk) {
    if (heads == 0 || dim == 0) return hipSuccess;
    const int nq = n_qk > 0 ? n_qk : heads;
    if (dim <= kGdnWaves * kGdnRows) {
        hipLaunchKernelGGL(gdn_step_wg_kernel, dim3((dim + 63) / 64, heads), dim3(64 * kGdnWaves), 0, s, state, out, q,
                           k, v, gate, beta, dim, scale, nq);
        return hipGetLastError();
    }
    const int tpb = dim >= 256 ? 256 : ((dim + 63) / 64) * 64;
    hipLaunchKernelGGL(gdn_step_kernel, dim3(heads), dim3(tpb), 0, s, state, out, q, k, v, gate, beta, dim, scale, nq);
    return hipGetLastError();
}

bool gdn_scan_ok(int dim, int d_conv) { return (dim == 64 || dim == 128) && d_conv >= 2 && d_conv <= 9; }

hipError_t launch_gdn_scan(float *win, const float *kern, const float *qkv, float *cv, float *beta, float *gexp,
                           const float *dt_bias, const float *a, const float *z, const float *snorm, float *state,
                           float *out, float *fin, int nt, int d_conv, int channels, int dim, int n_qk, int n_v,
                           float eps, float scale, hipStream_t s) {
    if (!gdn_scan_ok(dim, d_conv) || n_qk < 1 || channels != (2 * n_qk + n_v) * dim) return hipErrorInvalidValue;
    if (nt == 0 || n_v == 0) return hipSuccess;
    hipLaunchKernelGGL(gdn_conv_norm_rows_kernel, dim3((channels / dim + kConvUnits) / kConvUnits, nt),
                       dim3(64 * kConvUnits), 0, s, win, kern, qkv, cv, d_conv, channels, dim, n_qk, eps, beta, gexp,
                       dt_bias, a, n_v);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // eight rows per lane: a 128-dim head on 16 lanes per column (32 waves),
    // a 64-dim one on 8 (8 waves); then, as rows of the grid after the v
    // heads' (dispatched last, so the scan's workgroups spread over the CUs
    // first), the window's workgroups, a channel per thread
    const int scan_bx = (dim == 128 ? 32 : 8) / kScanWaves, tpb = 64 * kScanWaves;
    const int win_by = ((channels + tpb - 1) / tpb + scan_bx - 1) / scan_bx;
    const dim3 grid(scan_bx, n_v + win_by);
    if (dim == 128)
        hipLaunchKernelGGL((gdn_scan_kernel<16, 8>), grid, dim3(tpb), 0, s, cv, beta, gexp, state, out, nt, channels,
                           n_qk, n_v, scale, win, qkv, d_conv);
    else
        hipLaunchKernelGGL((gdn_scan_kernel<8, 8>), grid, dim3(tpb), 0, s, cv, beta, gexp, state, out, nt, channels,
                           n_qk, n_v, scale, win, qkv, d_conv);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    // the gated rmsnorm of every token's head outputs (rmsnorm_kernel with z)
    return launch_rmsnorm_rows(fin, dim, out, dim, snorm, dim, nt * n_v, eps, s, nullptr, nullptr, z);
}

hipError_t launch_rope_freq(int mode, float *x, int rows, int n, const float *freqs, size_t pos, hipStream_t s) {
    if (rows == 0 || n < 2) return hipSuccess;
    hipLaunchKernelGGL(rope_freq_kernel, dim3(ops_grid((size_t)rows * (n / 2))), dim3(OPS_TPB), 0, s, mode, x, rows,
                       n, freqs, (double)pos);
    return hipGetLastError();
}

hipError_t launch_rope_imrope(float *x, int rows, int n, int n_rot, double theta_scale, size_t pos, hipStream_t s) {
    if (rows == 0 || n_rot < 2) return hipSuccess;
    const int nrot3 = (n_rot / 2 + 2) / 3;
    hipLaunchKernelGGL(rope_imrope_kernel, dim3(ops_grid((size_t)rows * nrot3)), dim3(OPS_TPB), 0, s, x, rows, n,
                       n_rot, theta_scale, (double)pos);
    return hipGetLastError();
}

bool attn_shape_ok(int hd, int group) {
    return (hd == 64 || hd == 128 || hd == 256 || hd == 512) && group >= 1 && group <= kAttnMaxGroup;
}

hipError_t launch_attn_rows(float *out, size_t out_st, float *soft, size_t soft_st, const float *q, size_t q_st,
                            const float *kc, const float *vc, int n_ctx, int rows, int n_head_kv, int hd, int group,
                            float kq_scale, hipStream_t s, const float *gz, int gzs, size_t gz_st, float *gated,
                            size_t gated_st) {
    if (n_ctx <= 0 || n_head_kv <= 0 || rows <= 0) return hipSuccess;
    const int n_last = n_ctx + rows - 1;
    if (!attn_shape_ok(hd, group) || n_last > softmax_max_len() || rows > 65535) return hipErrorInvalidValue;
    if (rows > 1 && hd <= 256) {
        // a prefill chunk: lane-per-position dots, blocks of qb queries whose
        // q rows and the 64 K rows fit 80 KB of LDS
        const size_t kbytes = (size_t)kLaneScoresPos * (hd + 1) * 4;
        const int qb = (int)std::max<size_t>(1, std::min<size_t>(8, (80 * 1024 - kbytes) / ((size_t)group * hd * 4)));
        const size_t lds = (size_t)qb * group * hd * 4 + kbytes;
        const dim3 gl((n_last + kLaneScoresPos - 1) / kLaneScoresPos, n_head_kv, (rows + qb - 1) / qb);
        hipError_t e = hipSuccess;
        auto go = [&](const void *k, auto launch) {
            if ((e = allow_lds(k, lds)) == hipSuccess) launch();
        };
        switch (hd) {
            case 64: go((const void *)attn_scores_lane_kernel<64>, [&] { hipLaunchKernelGGL(attn_scores_lane_kernel<64>, gl, dim3(OPS_TPB), lds, s, soft, q, kc, n_ctx, n_head_kv, group, q_st, soft_st, rows, qb); }); break;
            case 128: go((const void *)attn_scores_lane_kernel<128>, [&] { hipLaunchKernelGGL(attn_scores_lane_kernel<128>, gl, dim3(OPS_TPB), lds, s, soft, q, kc, n_ctx, n_head_kv, group, q_st, soft_st, rows, qb); }); break;
            default: go((const void *)attn_scores_lane_kernel<256>, [&] { hipLaunchKernelGGL(attn_scores_lane_kernel<256>, gl, dim3(OPS_TPB), lds, s, soft, q, kc, n_ctx, n_head_kv, group, q_st, soft_st, rows, qb); }); break;
        }
        if (e != hipSuccess) return e;
    } else {
        const dim3 gs((n_last + kScoresPPB - 1) / kScoresPPB, n_head_kv, rows);
        switch (hd) {
            case 64: hipLaunchKernelGGL(attn_scores_kernel<1>, gs, dim3(OPS_TPB), 0, s, soft, q, kc, n_ctx, n_head_kv, group, q_st, soft_st); break;
            case 128: hipLaunchKernelGGL(attn_scores_kernel<2>, gs, dim3(OPS_TPB), 0, s, soft, q, kc, n_ctx, n_head_kv, group, q_st, soft_st); break;
            case 256: hipLaunchKernelGGL(attn_scores_kernel<4>, gs, dim3(OPS_TPB), 0, s, soft, q, kc, n_ctx, n_head_kv, group, q_st, soft_st); break;
            default: hipLaunchKernelGGL(attn_scores_kernel<8>, gs, dim3(OPS_TPB), 0, s, soft, q, kc, n_ctx, n_head_kv, group, q_st, soft_st); break;
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (n_last <= kSmWaveMax)
        hipLaunchKernelGGL(softmax_wave_kernel, dim3((n_head_kv * group + OPS_TPB / 64 - 1) / (OPS_TPB / 64), rows),
                           dim3(OPS_TPB), 0, s, soft, soft, n_ctx, kq_scale, 1, soft_st, n_head_kv * group);
    else
        hipLaunchKernelGGL(softmax_kernel, dim3(n_head_kv * group, rows), dim3(OPS_TPB), 0, s, soft, soft, n_ctx,
                           kq_scale, 1, soft_st);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const PvStrides pst{soft_st, out_st, gz_st, gated_st};
    if (rows > 1) {
        // a prefill chunk: 16 / group queries per workgroup
#define UQ_PVR(G) hipLaunchKernelGGL(attn_pv_rows_kernel<G>, dim3(hd / 64, n_head_kv, (rows + 16 / G - 1) / (16 / G)), \
                                     dim3(kPvRowsWaves * 64), 0, s, out, soft, vc, n_ctx, n_head_kv, hd, rows, gz, gzs, \
                                     gated, pst)
        switch (group) {
            case 1: UQ_PVR(1); break;
            case 2: UQ_PVR(2); break;
            case 3: UQ_PVR(3); break;
            case 4: UQ_PVR(4); break;
            case 5: UQ_PVR(5); break;
            case 6: UQ_PVR(6); break;
            case 7: UQ_PVR(7); break;
            default: UQ_PVR(8); break;
        }
#undef UQ_PVR
        return hipGetLastError();
    }
    const dim3 gp(hd / 64, n_head_kv, rows);
#define UQ_PV(G) hipLaunchKernelGGL(attn_pv_kernel<G>, gp, dim3(pv_waves<G>() * 64), 0, s, out, soft, vc, n_ctx, \
                                    n_head_kv, hd, gz, gzs, gated, pst)
    switch (group) {
        case 1: UQ_PV(1); break;
        case 2: UQ_PV(2); break;
        case 3: UQ_PV(3); break;
        case 4: UQ_PV(4); break;
        case 5: UQ_PV(5); break;
        case 6: UQ_PV(6); break;
        case 7: UQ_PV(7); break;
        default: UQ_PV(8); break;
    }
#undef UQ_PV
    return hipGetLastError();
}

hipError_t launch_attn_decode(float *out, float *soft, const float *q, const float *kc, const float *vc, int n_ctx,
                              int n_head_kv, int hd, int group, float kq_scale, hipStream_t s, const float *gz,
                              int gzs, float *gated) {
    return launch_attn_rows(out, 0, soft, 0, q, 0, kc, vc, n_ctx, 1, n_head_kv, hd, group, kq_scale, s, gz, gzs, 0,
                            gated, 0);
}

hipError_t launch_gdn_gates(const float *beta_raw, const float *alpha, const float *dt_bias, const float *a,
                            float *beta, float *sp, float *gate, int n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(gdn_gates_kernel, dim3(ops_grid(n)), dim3(OPS_TPB), 0, s, beta_raw, alpha, dt_bias, a, beta, sp,
                       gate, n);
    return hipGetLastError();
}

hipError_t launch_conv_step(float *win, const float *kern_gguf, float *raw, float *act, int d_conv, int channels,
                            hipStream_t s) {
    if (d_conv < 1 || d_conv > 9) return hipErrorInvalidValue;
    if (channels == 0) return hipSuccess;
    hipLaunchKernelGGL(conv_step_kernel, dim3(ops_grid(channels)), dim3(OPS_TPB), 0, s, win, kern_gguf, raw, act,
                       d_conv, channels);
    return hipGetLastError();
}

hipError_t launch_mul_act(int op, float *out, const float *y, const float *z, int n, int zs, size_t total,
                          hipStream_t s) {
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(mul_act_kernel, dim3(ops_grid(total)), dim3(OPS_TPB), 0, s, op, out, y, z, n, zs, total);
    return hipGetLastError();
}

hipError_t launch_gdn_conv_norm(float *win, const float *kern_gguf, float *raw, float *act, int d_conv, int channels,
                                int hd, int n_qk, float eps, const float *beta_raw, const float *alpha,
                                const float *dt_bias, const float *a, float *beta, float *sp, float *gate, int n_v,
                                hipStream_t s) {
    if (d_conv < 1 || d_conv > 9 || hd < 1 || hd > kConvNormMaxHd || channels % hd || 2 * n_qk > channels / hd)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(gdn_conv_norm_kernel, dim3(channels / hd + 1), dim3(OPS_TPB), 0, s, win, kern_gguf, raw, act,
                       d_conv, channels, hd, n_qk, eps, beta_raw, alpha, dt_bias, a, beta, sp, gate, n_v);
    return hipGetLastError();
}

bool conv_norm_ok(int hd) { return hd >= 1 && hd <= kConvNormMaxHd; }

hipError_t launch_attn_qk_prep(const float *qfull, float *q_out, const float *k_raw, float *k_out, const float *wq,
                               const float *wk, int hd, int n_head, int n_head_kv, int n_rot, double theta_scale,
                               size_t pos, float eps, hipStream_t s, int rows) {
    if (hd < 1 || hd > kQkMaxHd || n_rot > hd || n_rot % 2 || rows > 65535) return hipErrorInvalidValue;
    if (n_head + n_head_kv == 0 || rows <= 0) return hipSuccess;
    // rows of consecutive tokens: qfull [2 n_head hd], q_out [n_head hd],
    // k_raw and k_out (cache rows) [n_head_kv hd]
    const QkStrides st{(size_t)2 * n_head * hd, (size_t)n_head * hd, (size_t)n_head_kv * hd, (size_t)n_head_kv * hd};
    hipLaunchKernelGGL(attn_qk_prep_kernel, dim3(n_head + n_head_kv, rows), dim3(OPS_TPB), 0, s, qfull, q_out, k_raw,
                       k_out, wq, wk, hd, n_head, n_rot, theta_scale, (double)pos, eps, st);
    return hipGetLastError();
}

hipError_t launch_add(float *out, const float *a, const float *b, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(add_kernel, dim3(ops_grid(n)), dim3(OPS_TPB), 0, s, out, a, b, n);
    return hipGetLastError();
}

int matmul_max_k() { return kWaveTreeMax; }

hipError_t launch_matmul_acc(float *acc, const float *a, const float *b, int m, int k, int n, hipStream_t s) {
    if (m == 0 || n == 0) return hipSuccess;
    if (k > kWaveTreeMax) return hipErrorInvalidValue;
    const size_t waves = (size_t)m * n, blocks = (waves + OPS_TPB / 64 - 1) / (OPS_TPB / 64);
    if (blocks > 0x7fffffffu) return hipErrorInvalidValue;
    hipLaunchKernelGGL(matmul_acc_kernel, dim3((unsigned)blocks), dim3(OPS_TPB), 0, s, acc, a, b, m, k, n);
    return hipGetLastError();
}

}  // namespace uq
