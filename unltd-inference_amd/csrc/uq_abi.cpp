// C ABI of libuq (include/uq.h): argument checks in the reference's order,
// device memory for the host-pointer mirrors, and kernel dispatch.
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "uq_internal.h"

namespace {

thread_local std::string g_err;

uq_status fail(uq_status s, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return s;
}

}  // namespace

uq_status uq::set_error(uq_status s, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return s;
}

namespace {

uq_status hip_fail(hipError_t e, const char *what) {
    return fail(UQ_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

#define UQ_HIP(call, what)                          \
    do {                                            \
        hipError_t e_ = (call);                     \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

// The library ships gfx950 code objects only.
uq_status check_device() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(UQ_ERR_NO_DEVICE, "no HIP device");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(UQ_ERR_NO_DEVICE, "hipGetDevice failed");
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) return fail(UQ_ERR_NO_DEVICE, "hipGetDeviceProperties failed");
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(UQ_ERR_NO_DEVICE, "device %d is %s; libuq is built for gfx950", dev, p.gcnArchName);
    return UQ_OK;
}

// One stream per calling thread for the host-pointer entry points.
struct ThreadStream {
    hipStream_t s = nullptr;
    int dev = -1;
    ~ThreadStream() {
        if (s) (void)hipStreamDestroy(s);
    }
};
thread_local ThreadStream g_ts;

uq_status thread_stream(hipStream_t *out) {
    int dev = 0;
    UQ_HIP(hipGetDevice(&dev), "hipGetDevice");
    if (!g_ts.s || g_ts.dev != dev) {
        if (g_ts.s) (void)hipStreamDestroy(g_ts.s);
        g_ts.s = nullptr;
        UQ_HIP(hipStreamCreateWithFlags(&g_ts.s, hipStreamNonBlocking), "hipStreamCreate");
        g_ts.dev = dev;
    }
    *out = g_ts.s;
    return UQ_OK;
}

struct DevBuf {
    void *p = nullptr;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    hipError_t alloc(size_t n) { return hipMalloc(&p, n ? n : 1); }
    template <class T>
    T *as() const {
        return (T *)p;
    }
};

size_t row_bytes_of(uq_dtype dt, size_t n) {
    switch (dt) {
    case UQ_F32: return n * 4;
    case UQ_F16: return n * 2;
    case UQ_Q8_0: return n % 32 ? 0 : n / 32 * 34;
    case UQ_Q4_K: return n % 256 ? 0 : n / 256 * 144;
    case UQ_Q6_K: return n % 256 ? 0 : n / 256 * 210;
    default: return 0;
    }
}

const char *dtype_name(uq_dtype d) {
    switch (d) {
    case UQ_F32: return "F32";
    case UQ_F16: return "F16";
    case UQ_Q8_0: return "Q8_0";
    case UQ_Q4_K: return "Q4K";
    case UQ_Q6_K: return "Q6K";
    default: return "unknown";
    }
}

// gemv_quant's checks (quants.rs:430-452); Q8_0 accepted (closed form).
uq_status check_gemv_quant(const char *fn, size_t out_len, size_t x_len, size_t w_len, size_t dim_in,
                           size_t dim_out, uq_dtype dt, size_t *rb) {
    if (out_len != dim_out) return fail(UQ_ERR_LEN, "%s: len(out) %zu != dim_out %zu", fn, out_len, dim_out);
    if (x_len < dim_in) return fail(UQ_ERR_LEN, "%s: len(x) %zu < dim_in %zu", fn, x_len, dim_in);
    switch (dt) {
    case UQ_F32: *rb = dim_in * 4; break;
    case UQ_Q4_K:
    case UQ_Q6_K:
        if (dim_in % 256) return fail(UQ_ERR_BLOCK_MULTIPLE, "%s: dim_in %zu is not a multiple of 256", fn, dim_in);
        *rb = row_bytes_of(dt, dim_in);
        break;
    case UQ_Q8_0:
        if (dim_in % 32) return fail(UQ_ERR_BLOCK_MULTIPLE, "%s: dim_in %zu is not a multiple of 32", fn, dim_in);
        *rb = row_bytes_of(dt, dim_in);
        break;
    default: return fail(UQ_ERR_DTYPE, "%s: dtype %s has no dot kernel", fn, dtype_name(dt));
    }
    if (dim_out && *rb > SIZE_MAX / dim_out) return fail(UQ_ERR_LEN, "%s: size overflow", fn);
    if (w_len != *rb * dim_out)
        return fail(UQ_ERR_LEN, "%s: len(w) %zu != row_bytes %zu * dim_out %zu", fn, w_len, *rb, dim_out);
    if (dim_in > (size_t)INT_MAX || dim_out > (size_t)INT_MAX)
        return fail(UQ_ERR_ARG, "%s: dimensions above INT_MAX are not supported", fn);
    return UQ_OK;
}

bool bad_ptr(const void *p, size_t len) { return p == nullptr && len != 0; }

uq_weights_s *handle(uq_weights w) {
    return (w && w->magic == UQ_WEIGHTS_MAGIC) ? w : nullptr;
}

// Host-pointer GEMV shared by uq_gemv_quant / uq_gemv_quant_q8k.
uq_status host_gemv(bool q8k, float *out, const float *x, const uint8_t *w, size_t w_len, size_t dim_in,
                    size_t dim_out, size_t rb, uq_dtype dt) {
    if (dim_out == 0) return UQ_OK;
    if (dim_in == 0) {  // empty dot = 0 for every row (pairwise_sum of nothing)
        std::memset(out, 0, dim_out * sizeof(float));
        return UQ_OK;
    }
    uq_status st = check_device();
    if (st) return st;
    hipStream_t s;
    if ((st = thread_stream(&s))) return st;
    DevBuf dw, dx, dy;
    UQ_HIP(dw.alloc(w_len + UQ_WEIGHT_PAD), "hipMalloc(w)");
    UQ_HIP(dx.alloc(dim_in * 4), "hipMalloc(x)");
    UQ_HIP(dy.alloc(dim_out * 4), "hipMalloc(out)");
    UQ_HIP(hipMemcpyAsync(dw.p, w, w_len, hipMemcpyHostToDevice, s), "copy w");
    UQ_HIP(hipMemsetAsync(dw.as<uint8_t>() + w_len, 0, UQ_WEIGHT_PAD, s), "pad w");
    UQ_HIP(hipMemcpyAsync(dx.p, x, dim_in * 4, hipMemcpyHostToDevice, s), "copy x");
    const uq::WeightsView v{dw.as<uint8_t>(), dt, (int)dim_in, (int)dim_out, rb};
    UQ_HIP(q8k ? uq::launch_gemv_q8k(v, dx.as<float>(), dy.as<float>(), s)
               : uq::launch_gemv(v, dx.as<float>(), dy.as<float>(), s),
           q8k ? "gemv_quant_q8k launch" : "gemv_quant launch");
    UQ_HIP(hipMemcpyAsync(out, dy.p, dim_out * 4, hipMemcpyDeviceToHost, s), "copy out");
    UQ_HIP(hipStreamSynchronize(s), "synchronize");
    return UQ_OK;
}

uq_status host_dequant(const char *fn, uq_dtype dt, float *out, size_t out_len, const uint8_t *w,
                       size_t w_len) {
    const size_t be = dt == UQ_Q8_0 ? 32 : 256, bb = row_bytes_of(dt, be);
    if (bad_ptr(out, out_len) || bad_ptr(w, w_len)) return fail(UQ_ERR_ARG, "%s: null pointer", fn);
    if (w_len != out_len / be * bb)
        return fail(UQ_ERR_LEN, "%s: len(w) %zu != blocks for len(out) %zu", fn, w_len, out_len);
    if (out_len % be) return fail(UQ_ERR_LEN, "%s: len(out) %zu is not a multiple of %zu", fn, out_len, be);
    if (out_len == 0) return UQ_OK;
    uq_status st = check_device();
    if (st) return st;
    hipStream_t s;
    if ((st = thread_stream(&s))) return st;
    DevBuf dw, dy;
    UQ_HIP(dw.alloc(w_len), "hipMalloc(w)");
    UQ_HIP(dy.alloc(out_len * 4), "hipMalloc(out)");
    UQ_HIP(hipMemcpyAsync(dw.p, w, w_len, hipMemcpyHostToDevice, s), "copy w");
    UQ_HIP(uq::launch_dequant(dt, dw.as<uint8_t>(), out_len, dy.as<float>(), s), "dequantize launch");
    UQ_HIP(hipMemcpyAsync(out, dy.p, out_len * 4, hipMemcpyDeviceToHost, s), "copy out");
    UQ_HIP(hipStreamSynchronize(s), "synchronize");
    return UQ_OK;
}

uq_status host_unpack(uq_dtype dt, const uint8_t *w, size_t nblocks, void *q, void *sc, uint8_t *m, float *d,
                      float *dmin) {
    if (nblocks == 0) return UQ_OK;
    const size_t bb = row_bytes_of(dt, dt == UQ_Q8_0 ? 32 : 256);
    const size_t nq = nblocks * (dt == UQ_Q8_0 ? 32 : 256);
    const size_t nsc = dt == UQ_Q4_K ? nblocks * 8 : (dt == UQ_Q6_K ? nblocks * 16 : 0);
    uq_status st = check_device();
    if (st) return st;
    hipStream_t s;
    if ((st = thread_stream(&s))) return st;
    DevBuf dw, dq, dsc, dm, dd, ddm;
    UQ_HIP(dw.alloc(nblocks * bb), "hipMalloc(w)");
    UQ_HIP(dq.alloc(nq), "hipMalloc(q)");
    UQ_HIP(dsc.alloc(nsc), "hipMalloc(sc)");
    UQ_HIP(dm.alloc(nsc), "hipMalloc(m)");
    UQ_HIP(dd.alloc(nblocks * 4), "hipMalloc(d)");
    UQ_HIP(ddm.alloc(nblocks * 4), "hipMalloc(dmin)");
    UQ_HIP(hipMemcpyAsync(dw.p, w, nblocks * bb, hipMemcpyHostToDevice, s), "copy w");
    UQ_HIP(uq::launch_unpack(dt, dw.as<uint8_t>(), nblocks, dq.p, dsc.p, dm.as<uint8_t>(), dd.as<float>(),
                             ddm.as<float>(), s),
           "unpack launch");
    UQ_HIP(hipMemcpyAsync(q, dq.p, nq, hipMemcpyDeviceToHost, s), "copy q");
    if (nsc) UQ_HIP(hipMemcpyAsync(sc, dsc.p, nsc, hipMemcpyDeviceToHost, s), "copy sc");
    if (dt == UQ_Q4_K) UQ_HIP(hipMemcpyAsync(m, dm.p, nsc, hipMemcpyDeviceToHost, s), "copy m");
    UQ_HIP(hipMemcpyAsync(d, dd.p, nblocks * 4, hipMemcpyDeviceToHost, s), "copy d");
    if (dt == UQ_Q4_K) UQ_HIP(hipMemcpyAsync(dmin, ddm.p, nblocks * 4, hipMemcpyDeviceToHost, s), "copy dmin");
    UQ_HIP(hipStreamSynchronize(s), "synchronize");
    return UQ_OK;
}

}  // namespace

uq_status uq::host_stream(hipStream_t *s) {
    const uq_status st = check_device();
    return st ? st : thread_stream(s);
}

uq_status uq::hip_error(hipError_t e, const char *what) { return hip_fail(e, what); }


extern "C" {

const char *uq_last_error(void) { return g_err.c_str(); }

const char *uq_status_name(uq_status s) {
    switch (s) {
    case UQ_OK: return "UQ_OK";
    case UQ_ERR_LEN: return "UQ_ERR_LEN";
    case UQ_ERR_BLOCK_MULTIPLE: return "UQ_ERR_BLOCK_MULTIPLE";
    case UQ_ERR_DTYPE: return "UQ_ERR_DTYPE";
    case UQ_ERR_ARG: return "UQ_ERR_ARG";
    case UQ_ERR_HIP: return "UQ_ERR_HIP";
    case UQ_ERR_NO_DEVICE: return "UQ_ERR_NO_DEVICE";
    case UQ_ERR_TOKEN: return "UQ_ERR_TOKEN";
    case UQ_ERR_FILE: return "UQ_ERR_FILE";
    case UQ_ERR_MAGIC: return "UQ_ERR_MAGIC";
    case UQ_ERR_VERSION: return "UQ_ERR_VERSION";
    case UQ_ERR_TENSOR_BOUNDS: return "UQ_ERR_TENSOR_BOUNDS";
    case UQ_ERR_TENSOR_OVERLAP: return "UQ_ERR_TENSOR_OVERLAP";
    case UQ_ERR_TENSOR_ALIGN: return "UQ_ERR_TENSOR_ALIGN";
    case UQ_ERR_GGML_TYPE: return "UQ_ERR_GGML_TYPE";
    case UQ_ERR_MISSING_TENSOR: return "UQ_ERR_MISSING_TENSOR";
    case UQ_ERR_ELEMENT_COUNT: return "UQ_ERR_ELEMENT_COUNT";
    case UQ_ERR_IO: return "UQ_ERR_IO";
    default: return "UQ_ERR_UNKNOWN";
    }
}

size_t uq_row_bytes(uq_dtype dtype, size_t dim_in) { return row_bytes_of(dtype, dim_in); }

uq_status uq_gemv_quant(float *out, size_t out_len, const float *x, size_t x_len, const uint8_t *w,
                        size_t w_len, size_t dim_in, size_t dim_out, uq_dtype dtype) {
    size_t rb = 0;
    uq_status st = check_gemv_quant("gemv_quant", out_len, x_len, w_len, dim_in, dim_out, dtype, &rb);
    if (st) return st;
    if (bad_ptr(out, out_len) || bad_ptr(x, x_len) || bad_ptr(w, w_len))
        return fail(UQ_ERR_ARG, "gemv_quant: null pointer");
    return host_gemv(false, out, x, w, w_len, dim_in, dim_out, rb, dtype);
}

uq_status uq_gemv_quant_q8k(float *out, size_t out_len, const float *x, size_t x_len, const uint8_t *w,
                            size_t w_len, size_t dim_in, size_t dim_out, uq_dtype dtype) {
    // quants.rs:482-505: lengths, then the dtype match (Q4_K/Q6_K only, with
    // the multiple-of-256 check inside), then len(w)
    if (out_len != dim_out)
        return fail(UQ_ERR_LEN, "gemv_quant_q8k: len(out) %zu != dim_out %zu", out_len, dim_out);
    if (x_len < dim_in) return fail(UQ_ERR_LEN, "gemv_quant_q8k: len(x) %zu < dim_in %zu", x_len, dim_in);
    if (dtype != UQ_Q4_K && dtype != UQ_Q6_K)
        return fail(UQ_ERR_DTYPE, "gemv_quant_q8k: dtype %s does not use the Q8_K dot", dtype_name(dtype));
    size_t rb = 0;
    uq_status st = check_gemv_quant("gemv_quant_q8k", out_len, x_len, w_len, dim_in, dim_out, dtype, &rb);
    if (st) return st;
    if (bad_ptr(out, out_len) || bad_ptr(x, x_len) || bad_ptr(w, w_len))
        return fail(UQ_ERR_ARG, "gemv_quant_q8k: null pointer");
    return host_gemv(true, out, x, w, w_len, dim_in, dim_out, rb, dtype);
}

uq_status uq_quantize_q8_k(uq_q8k_block *out, size_t out_blocks, const float *x, size_t x_len) {
    if (x_len % 256) return fail(UQ_ERR_BLOCK_MULTIPLE, "quantize_q8_k: len %zu is not a multiple of 256", x_len);
    if (out_blocks != x_len / 256)
        return fail(UQ_ERR_LEN, "quantize_q8_k: out holds %zu blocks, x has %zu", out_blocks, x_len / 256);
    if (bad_ptr(out, out_blocks) || bad_ptr(x, x_len)) return fail(UQ_ERR_ARG, "quantize_q8_k: null pointer");
    if (x_len == 0) return UQ_OK;
    uq_status st = check_device();
    if (st) return st;
    hipStream_t s;
    if ((st = thread_stream(&s))) return st;
    DevBuf dx, dq;
    UQ_HIP(dx.alloc(x_len * 4), "hipMalloc(x)");
    UQ_HIP(dq.alloc(out_blocks * sizeof(uq_q8k_block)), "hipMalloc(out)");
    UQ_HIP(hipMemcpyAsync(dx.p, x, x_len * 4, hipMemcpyHostToDevice, s), "copy x");
    UQ_HIP(uq::launch_quantize_q8k(dx.as<float>(), x_len, dq.as<uq_q8k_block>(), s), "quantize launch");
    UQ_HIP(hipMemcpyAsync(out, dq.p, out_blocks * sizeof(uq_q8k_block), hipMemcpyDeviceToHost, s), "copy out");
    UQ_HIP(hipStreamSynchronize(s), "synchronize");
    return UQ_OK;
}

uq_status uq_dequantize_q4_k(float *out, size_t out_len, const uint8_t *w, size_t w_len) {
    return host_dequant("dequantize_q4_k", UQ_Q4_K, out, out_len, w, w_len);
}
uq_status uq_dequantize_q6_k(float *out, size_t out_len, const uint8_t *w, size_t w_len) {
    return host_dequant("dequantize_q6_k", UQ_Q6_K, out, out_len, w, w_len);
}
uq_status uq_dequantize_q8_0(float *out, size_t out_len, const uint8_t *w, size_t w_len) {
    return host_dequant("dequantize_q8_0", UQ_Q8_0, out, out_len, w, w_len);
}

uq_status uq_unpack_q4_k(const uint8_t *w, size_t nblocks, uint8_t *q, uint8_t *sc, uint8_t *m, float *d,
                         float *dmin) {
    if (nblocks && (!w || !q || !sc || !m || !d || !dmin)) return fail(UQ_ERR_ARG, "unpack_q4_k: null pointer");
    return host_unpack(UQ_Q4_K, w, nblocks, q, sc, m, d, dmin);
}
uq_status uq_unpack_q6_k(const uint8_t *w, size_t nblocks, uint8_t *q, int8_t *sc, float *d) {
    if (nblocks && (!w || !q || !sc || !d)) return fail(UQ_ERR_ARG, "unpack_q6_k: null pointer");
    return host_unpack(UQ_Q6_K, w, nblocks, q, sc, nullptr, d, nullptr);
}
uq_status uq_unpack_q8_0(const uint8_t *w, size_t nblocks, int8_t *q, float *d) {
    if (nblocks && (!w || !q || !d)) return fail(UQ_ERR_ARG, "unpack_q8_0: null pointer");
    return host_unpack(UQ_Q8_0, w, nblocks, q, nullptr, nullptr, d, nullptr);
}

uq_status uq_f16_to_f32(float *out, const uint16_t *h, size_t n) {
    if (bad_ptr(out, n) || bad_ptr(h, n)) return fail(UQ_ERR_ARG, "f16_to_f32: null pointer");
    if (n == 0) return UQ_OK;
    uq_status st = check_device();
    if (st) return st;
    hipStream_t s;
    if ((st = thread_stream(&s))) return st;
    DevBuf dh, dy;
    UQ_HIP(dh.alloc(n * 2), "hipMalloc(h)");
    UQ_HIP(dy.alloc(n * 4), "hipMalloc(out)");
    UQ_HIP(hipMemcpyAsync(dh.p, h, n * 2, hipMemcpyHostToDevice, s), "copy h");
    UQ_HIP(uq::launch_f16_to_f32(dh.as<uint16_t>(), n, dy.as<float>(), s), "f16 launch");
    UQ_HIP(hipMemcpyAsync(out, dy.p, n * 4, hipMemcpyDeviceToHost, s), "copy out");
    UQ_HIP(hipStreamSynchronize(s), "synchronize");
    return UQ_OK;
}

uq_status uq_swiglu(float *out, const float *gate, const float *up, size_t n) {
    if (bad_ptr(out, n) || bad_ptr(gate, n) || bad_ptr(up, n)) return fail(UQ_ERR_ARG, "swiglu: null pointer");
    if (n == 0) return UQ_OK;
    uq_status st = check_device();
    if (st) return st;
    hipStream_t s;
    if ((st = thread_stream(&s))) return st;
    DevBuf dg, du, dy;
    UQ_HIP(dg.alloc(n * 4), "hipMalloc(gate)");
    UQ_HIP(du.alloc(n * 4), "hipMalloc(up)");
    UQ_HIP(dy.alloc(n * 4), "hipMalloc(out)");
    UQ_HIP(hipMemcpyAsync(dg.p, gate, n * 4, hipMemcpyHostToDevice, s), "copy gate");
    UQ_HIP(hipMemcpyAsync(du.p, up, n * 4, hipMemcpyHostToDevice, s), "copy up");
    UQ_HIP(uq::launch_swiglu(dg.as<float>(), du.as<float>(), n, dy.as<float>(), s), "swiglu launch");
    UQ_HIP(hipMemcpyAsync(out, dy.p, n * 4, hipMemcpyDeviceToHost, s), "copy out");
    UQ_HIP(hipStreamSynchronize(s), "synchronize");
    return UQ_OK;
}

// ----------------------------------------------------------- device API

uq_status uq_weights_upload(uq_weights *out, const void *bytes, size_t nbytes, uq_dtype dtype, size_t dim_in,
                            size_t dim_out) {
    if (!out) return fail(UQ_ERR_ARG, "weights_upload: null handle pointer");
    *out = nullptr;
    if (bad_ptr(bytes, nbytes)) return fail(UQ_ERR_ARG, "weights_upload: null bytes");
    size_t rb = 0;
    switch (dtype) {
    case UQ_F32: rb = dim_in * 4; break;
    case UQ_Q4_K:
    case UQ_Q6_K:
        if (dim_in % 256) return fail(UQ_ERR_BLOCK_MULTIPLE, "weights_upload: dim_in %zu is not a multiple of 256", dim_in);
        rb = row_bytes_of(dtype, dim_in);
        break;
    case UQ_Q8_0:
        if (dim_in % 32) return fail(UQ_ERR_BLOCK_MULTIPLE, "weights_upload: dim_in %zu is not a multiple of 32", dim_in);
        rb = row_bytes_of(dtype, dim_in);
        break;
    default: return fail(UQ_ERR_DTYPE, "weights_upload: dtype %s has no dot kernel", dtype_name(dtype));
    }
    if (dim_out && rb > SIZE_MAX / dim_out) return fail(UQ_ERR_LEN, "weights_upload: size overflow");
    if (nbytes != rb * dim_out)
        return fail(UQ_ERR_LEN, "weights_upload: %zu bytes != row_bytes %zu * dim_out %zu", nbytes, rb, dim_out);
    if (dim_in > (size_t)INT_MAX || dim_out > (size_t)INT_MAX)
        return fail(UQ_ERR_ARG, "weights_upload: dimensions above INT_MAX are not supported");
    uq_status st = check_device();
    if (st) return st;
    uq_weights_s *w = new uq_weights_s();
    w->magic = UQ_WEIGHTS_MAGIC;
    (void)hipGetDevice(&w->device);
    w->dtype = dtype;
    w->dim_in = dim_in;
    w->dim_out = dim_out;
    w->row_bytes = rb;
    w->nbytes = nbytes;
    hipError_t e = hipMalloc((void **)&w->d_bytes, nbytes + UQ_WEIGHT_PAD);
    if (e == hipSuccess && nbytes) e = hipMemcpy(w->d_bytes, bytes, nbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(w->d_bytes + nbytes, 0, UQ_WEIGHT_PAD);
    if (e != hipSuccess) {
        if (w->d_bytes) (void)hipFree(w->d_bytes);
        delete w;
        return hip_fail(e, "weights_upload");
    }
    *out = w;
    return UQ_OK;
}

uq_status uq_weights_free(uq_weights wh) {
    uq_weights_s *w = handle(wh);
    if (!w) return fail(UQ_ERR_ARG, "weights_free: invalid handle");
    w->magic = 0;
    hipError_t e = hipFree(w->d_bytes);
    delete w;
    if (e != hipSuccess) return hip_fail(e, "weights_free");
    return UQ_OK;
}

uq_status uq_weights_info(uq_weights wh, uq_dtype *dtype, size_t *dim_in, size_t *dim_out, size_t *nbytes) {
    uq_weights_s *w = handle(wh);
    if (!w) return fail(UQ_ERR_ARG, "weights_info: invalid handle");
    if (dtype) *dtype = w->dtype;
    if (dim_in) *dim_in = w->dim_in;
    if (dim_out) *dim_out = w->dim_out;
    if (nbytes) *nbytes = w->nbytes;
    return UQ_OK;
}

uq_status uq_gemv(uq_weights wh, const float *d_x, float *d_y, void *stream) {
    uq_weights_s *w = handle(wh);
    if (!w) return fail(UQ_ERR_ARG, "gemv: invalid handle");
    if (w->dim_out == 0) return UQ_OK;
    if (!d_y || (!d_x && w->dim_in)) return fail(UQ_ERR_ARG, "gemv: null device pointer");
    UQ_HIP(uq::launch_gemv(uq::view(*w), d_x, d_y, (hipStream_t)stream), "gemv launch");
    return UQ_OK;
}

// Shared validation of the batched GEMV entry points: fills v[0..count).
static uq_status batch_views(const char *fn, const uq_weights *whs, float *const *d_y, size_t count,
                             const float *d_x, bool q8k, uq::WeightsView *v) {
    if (!whs || !d_y) return fail(UQ_ERR_ARG, "%s: null argument", fn);
    if (count > UQ_GEMV_BATCH_MAX) return fail(UQ_ERR_ARG, "%s: count %zu above %d", fn, count, UQ_GEMV_BATCH_MAX);
    uq_weights_s *first = nullptr;
    size_t rows = 0;
    for (size_t i = 0; i < count; i++) {
        uq_weights_s *w = handle(whs[i]);
        if (!w) return fail(UQ_ERR_ARG, "%s: invalid handle %zu", fn, i);
        if (!first) first = w;
        if (q8k && w->dtype != UQ_Q4_K && w->dtype != UQ_Q6_K)
            return fail(UQ_ERR_DTYPE, "%s: dtype %s does not use the Q8_K dot", fn, dtype_name(w->dtype));
        if (w->dtype != first->dtype || w->dim_in != first->dim_in)
            return fail(UQ_ERR_LEN, "%s: weights %zu differ from weights 0 in dtype or dim_in", fn, i);
        if (w->device != first->device) return fail(UQ_ERR_ARG, "%s: weights on different devices", fn);
        if (w->dim_out && !d_y[i]) return fail(UQ_ERR_ARG, "%s: null output %zu", fn, i);
        v[i] = uq::view(*w);
        rows += w->dim_out;
    }
    if (first && !d_x && first->dim_in) return fail(UQ_ERR_ARG, "%s: null device pointer", fn);
    if (rows > (size_t)INT_MAX) return fail(UQ_ERR_ARG, "%s: more than INT_MAX rows", fn);
    return UQ_OK;
}

uq_status uq_gemv_batch(const uq_weights *whs, float *const *d_y, size_t count, const float *d_x, void *stream) {
    uq::WeightsView v[UQ_GEMV_BATCH_MAX];
    uq_status st = batch_views("gemv_batch", whs, d_y, count, d_x, false, v);
    if (st != UQ_OK || count == 0) return st;
    UQ_HIP(uq::launch_gemv_batch(v, (int)count, d_x, d_y, (hipStream_t)stream), "gemv_batch launch");
    return UQ_OK;
}

uq_status uq_gemv_q8k_batch(const uq_weights *whs, float *const *d_y, size_t count, const float *d_x,
                            void *stream) {
    uq::WeightsView v[UQ_GEMV_BATCH_MAX];
    uq_status st = batch_views("gemv_q8k_batch", whs, d_y, count, d_x, true, v);
    if (st != UQ_OK || count == 0) return st;
    UQ_HIP(uq::launch_gemv_q8k_batch(v, (int)count, d_x, d_y, (hipStream_t)stream), "gemv_q8k_batch launch");
    return UQ_OK;
}

uq_status uq_swiglu_d(float *d_out, const float *d_gate, const float *d_up, size_t n, void *stream) {
    if (n == 0) return UQ_OK;
    if (!d_out || !d_gate || !d_up) return fail(UQ_ERR_ARG, "swiglu_d: null device pointer");
    UQ_HIP(uq::launch_swiglu(d_gate, d_up, n, d_out, (hipStream_t)stream), "swiglu_d launch");
    return UQ_OK;
}

uq_status uq_ffn_swiglu_q8k(uq_weights gh, uq_weights uh, uq_weights dh, const float *d_x, float *d_g, float *d_u,
                            float *d_h, float *d_y, void *stream) {
    return uq::ffn_swiglu_q8k_sum(gh, uh, dh, d_x, d_g, d_u, d_h, d_y, nullptr, nullptr, stream);
}

}  // extern "C"

// uq_ffn_swiglu_q8k; with d_ysum set, the down projection also writes
// d_ysum = d_add + d_y (the layer's residual sum, in the same launch).
uq_status uq::ffn_swiglu_q8k_sum(uq_weights gh, uq_weights uh, uq_weights dh, const float *d_x, float *d_g,
                                 float *d_u, float *d_h, float *d_y, const float *d_add, float *d_ysum,
                                 void *stream) {
    uq_weights_s *g = handle(gh), *u = handle(uh), *dn = handle(dh);
    if (!g || !u || !dn) return fail(UQ_ERR_ARG, "ffn_swiglu_q8k: invalid handle");
    for (uq_weights_s *w : {g, u, dn})
        if (w->dtype != UQ_Q4_K && w->dtype != UQ_Q6_K)
            return fail(UQ_ERR_DTYPE, "ffn_swiglu_q8k: dtype %s does not use the Q8_K dot", dtype_name(w->dtype));
    if (g->dtype != u->dtype || g->dim_in != u->dim_in || g->dim_out != u->dim_out)
        return fail(UQ_ERR_LEN, "ffn_swiglu_q8k: gate and up differ in dtype or shape");
    if (dn->dim_in != g->dim_out)
        return fail(UQ_ERR_LEN, "ffn_swiglu_q8k: down dim_in %zu != n_ff %zu", dn->dim_in, g->dim_out);
    if (!d_x || !d_g || !d_u || !d_h || !d_y) return fail(UQ_ERR_ARG, "ffn_swiglu_q8k: null device pointer");
    const hipStream_t s = (hipStream_t)stream;
    const uq::WeightsView gu[2] = {uq::view(*g), uq::view(*u)};
    bool fused = false;
    UQ_HIP(uq::launch_q8k_gate_up(gu[0], gu[1], d_x, d_g, d_u, d_h, s, &fused), "ffn_q8k gate/up/swiglu launch");
    if (!fused) {
        float *const gy[2] = {d_g, d_u};
        UQ_HIP(uq::launch_gemv_q8k_batch(gu, 2, d_x, gy, s), "ffn_q8k gate/up launch");
        UQ_HIP(uq::launch_swiglu(d_g, d_u, g->dim_out, d_h, s), "ffn_q8k swiglu launch");
    }
    if (d_ysum)
        UQ_HIP(uq::launch_gemv_q8k_sum(uq::view(*dn), d_h, d_y, d_add, d_ysum, s), "ffn_q8k down launch");
    else
        UQ_HIP(uq::launch_gemv_q8k(uq::view(*dn), d_h, d_y, s), "ffn_q8k down launch");
    return UQ_OK;
}

extern "C" {

uq_status uq_gemv_q8k(uq_weights wh, const float *d_x, float *d_y, void *stream) {
    uq_weights_s *w = handle(wh);
    if (!w) return fail(UQ_ERR_ARG, "gemv_q8k: invalid handle");
    if (w->dtype != UQ_Q4_K && w->dtype != UQ_Q6_K)
        return fail(UQ_ERR_DTYPE, "gemv_q8k: dtype %s does not use the Q8_K dot", dtype_name(w->dtype));
    if (w->dim_out == 0) return UQ_OK;
    if (!d_y || (!d_x && w->dim_in)) return fail(UQ_ERR_ARG, "gemv_q8k: null device pointer");
    UQ_HIP(uq::launch_gemv_q8k(uq::view(*w), d_x, d_y, (hipStream_t)stream), "gemv_q8k launch");
    return UQ_OK;
}

uq_status uq_gemm(uq_weights wh, size_t m_rows, const float *d_x, float *d_y, void *stream) {
    uq_weights_s *w = handle(wh);
    if (!w) return fail(UQ_ERR_ARG, "gemm: invalid handle");
    if (m_rows == 0 || w->dim_out == 0) return UQ_OK;
    if (m_rows > (size_t)INT_MAX) return fail(UQ_ERR_ARG, "gemm: m_rows above INT_MAX");
    if (!d_y || !d_x) return fail(UQ_ERR_ARG, "gemm: null device pointer");
    UQ_HIP(uq::launch_gemm(uq::view(*w), (int)m_rows, d_x, d_y, (hipStream_t)stream), "gemm launch");
    return UQ_OK;
}

uq_status uq_gemm_q8k(uq_weights wh, size_t m_rows, const float *d_x, float *d_y, void *stream) {
    uq_weights_s *w = handle(wh);
    if (!w) return fail(UQ_ERR_ARG, "gemm_q8k: invalid handle");
    if (w->dtype != UQ_Q4_K && w->dtype != UQ_Q6_K)
        return fail(UQ_ERR_DTYPE, "gemm_q8k: dtype %s does not use the Q8_K dot", dtype_name(w->dtype));
    if (m_rows == 0 || w->dim_out == 0) return UQ_OK;
    if (m_rows > (size_t)INT_MAX / 2) return fail(UQ_ERR_ARG, "gemm_q8k: m_rows above INT_MAX / 2");
    if (!d_y || (!d_x && w->dim_in)) return fail(UQ_ERR_ARG, "gemm_q8k: null device pointer");
    if (w->dim_in / 256 > 65535) return fail(UQ_ERR_ARG, "gemm_q8k: dim_in above 65535 blocks of 256");
    UQ_HIP(uq::launch_gemm_q8k(uq::view(*w), (int)m_rows, d_x, d_y, (hipStream_t)stream), "gemm_q8k launch");
    return UQ_OK;
}

uq_status uq_gemm_q8k_batch(const uq_weights *whs, float *const *d_y, size_t count, size_t m_rows, const float *d_x,
                            void *stream) {
    static_assert(UQ_GEMM_Q8K_BATCH_MAX == uq::kGemmQ8kBatchMax, "batch bound");
    if (count > UQ_GEMM_Q8K_BATCH_MAX)
        return fail(UQ_ERR_ARG, "gemm_q8k_batch: count %zu above %d", count, UQ_GEMM_Q8K_BATCH_MAX);
    uq::WeightsView v[UQ_GEMV_BATCH_MAX];
    uq_status st = batch_views("gemm_q8k_batch", whs, d_y, count, d_x, true, v);
    if (st != UQ_OK || count == 0 || m_rows == 0) return st;
    if (m_rows > (size_t)INT_MAX / 2) return fail(UQ_ERR_ARG, "gemm_q8k_batch: m_rows above INT_MAX / 2");
    if (v[0].dim_in / 256 > 65535) return fail(UQ_ERR_ARG, "gemm_q8k_batch: dim_in above 65535 blocks of 256");
    UQ_HIP(uq::launch_gemm_q8k_batch(v, (int)count, (int)m_rows, d_x, d_y, (hipStream_t)stream),
           "gemm_q8k_batch launch");
    return UQ_OK;
}

uq_status uq_gemm_static(uq_weights wh, size_t m_rows, const float *d_x, float *d_y, void *stream) {
    uq_weights_s *w = handle(wh);
    if (!w) return fail(UQ_ERR_ARG, "gemm_static: invalid handle");
    if (m_rows == 0 || w->dim_out == 0) return UQ_OK;
    if (m_rows > (size_t)INT_MAX) return fail(UQ_ERR_ARG, "gemm_static: m_rows above INT_MAX");
    if (!d_y || !d_x) return fail(UQ_ERR_ARG, "gemm_static: null device pointer");
    const uq::WeightsView v = uq::view(*w);
    const size_t need = uq::gemm_ws_bytes(v, (int)m_rows);
    if (need > UQ_GEMM_SCRATCH_BYTES)
        return fail(UQ_ERR_ARG, "gemm_static: workspace of %zu bytes for m_rows %zu exceeds the fixed %u bytes",
                    need, m_rows, (unsigned)UQ_GEMM_SCRATCH_BYTES);
    UQ_HIP(uq::launch_gemm_static(v, (int)m_rows, d_x, d_y, (hipStream_t)stream), "gemm_static launch");
    return UQ_OK;
}

uq_status uq_ffn_swiglu(uq_weights gh, uq_weights uh, uq_weights dh, const float *d_x, float *d_h, float *d_y,
                        void *stream) {
    uq_weights_s *g = handle(gh), *u = handle(uh), *dn = handle(dh);
    if (!g || !u || !dn) return fail(UQ_ERR_ARG, "ffn_swiglu: invalid handle");
    if (g->dtype != u->dtype || g->dim_in != u->dim_in || g->dim_out != u->dim_out)
        return fail(UQ_ERR_LEN, "ffn_swiglu: gate and up differ in dtype or shape");
    if (dn->dim_in != g->dim_out)
        return fail(UQ_ERR_LEN, "ffn_swiglu: down dim_in %zu != n_ff %zu", dn->dim_in, g->dim_out);
    if (!d_x || !d_h || !d_y) return fail(UQ_ERR_ARG, "ffn_swiglu: null device pointer");
    const hipStream_t s = (hipStream_t)stream;
    UQ_HIP(uq::launch_gate_up_swiglu(uq::view(*g), uq::view(*u), d_x, d_h, s), "ffn gate/up launch");
    UQ_HIP(uq::launch_gemv(uq::view(*dn), d_h, d_y, s), "ffn down launch");
    return UQ_OK;
}

uq_status uq_dequantize(uq_weights wh, float *d_out, void *stream) {
    uq_weights_s *w = handle(wh);
    if (!w) return fail(UQ_ERR_ARG, "dequantize: invalid handle");
    if (!d_out && w->nbytes) return fail(UQ_ERR_ARG, "dequantize: null device pointer");
    if (w->dtype == UQ_F32) {
        UQ_HIP(hipMemcpyAsync(d_out, w->d_bytes, w->nbytes, hipMemcpyDeviceToDevice, (hipStream_t)stream),
               "dequantize copy");
        return UQ_OK;
    }
    UQ_HIP(uq::launch_dequant(w->dtype, w->d_bytes, w->dim_in * w->dim_out, d_out, (hipStream_t)stream),
           "dequantize launch");
    return UQ_OK;
}

uq_status uq_embed(uq_weights wh, const uint32_t *tokens, size_t n_tokens, float *d_out, void *stream) {
    uq_weights_s *w = handle(wh);
    if (!w) return fail(UQ_ERR_ARG, "embed: invalid handle");
    if (n_tokens == 0) return UQ_OK;
    if (!tokens || !d_out) return fail(UQ_ERR_ARG, "embed: null pointer");
    for (size_t r = 0; r < n_tokens; r++)
        if (tokens[r] >= w->dim_out)
            return fail(UQ_ERR_TOKEN, "embed: token %u out of the vocabulary (0..%zu)", tokens[r], w->dim_out);
    UQ_HIP(uq::launch_embed(w->dtype, w->d_bytes, w->row_bytes, (int)w->dim_in, tokens, n_tokens, d_out,
                            (hipStream_t)stream),
           "embed launch");
    return UQ_OK;
}

uq_status uq_device_count(int *n) {
    if (!n) return fail(UQ_ERR_ARG, "device_count: null pointer");
    *n = 0;
    if (hipGetDeviceCount(n) != hipSuccess) *n = 0;
    return UQ_OK;
}

uq_status uq_device_name(char *buf, size_t len) {
    if (!buf || !len) return fail(UQ_ERR_ARG, "device_name: empty buffer");
    uq_status st = check_device();
    int dev = 0;
    hipDeviceProp_t p;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess) {
        buf[0] = 0;
        return st ? st : fail(UQ_ERR_NO_DEVICE, "device_name: no device");
    }
    snprintf(buf, len, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    return st;
}

uq_status uq_malloc(void **d_ptr, size_t nbytes) {
    if (!d_ptr) return fail(UQ_ERR_ARG, "malloc: null pointer");
    *d_ptr = nullptr;
    UQ_HIP(hipMalloc(d_ptr, nbytes ? nbytes : 1), "hipMalloc");
    return UQ_OK;
}

uq_status uq_free(void *d_ptr) {
    if (d_ptr) UQ_HIP(hipFree(d_ptr), "hipFree");
    return UQ_OK;
}

uq_status uq_memcpy_htod(void *d_dst, const void *src, size_t nbytes, void *stream) {
    if (!nbytes) return UQ_OK;
    UQ_HIP(hipMemcpyAsync(d_dst, src, nbytes, hipMemcpyHostToDevice, (hipStream_t)stream), "memcpy htod");
    return UQ_OK;
}

uq_status uq_memcpy_dtoh(void *dst, const void *d_src, size_t nbytes, void *stream) {
    if (!nbytes) return UQ_OK;
    UQ_HIP(hipMemcpyAsync(dst, d_src, nbytes, hipMemcpyDeviceToHost, (hipStream_t)stream), "memcpy dtoh");
    UQ_HIP(hipStreamSynchronize((hipStream_t)stream), "memcpy dtoh sync");
    return UQ_OK;
}

uq_status uq_memcpy_dtod(void *d_dst, const void *d_src, size_t nbytes, void *stream) {
    if (!nbytes) return UQ_OK;
    UQ_HIP(hipMemcpyAsync(d_dst, d_src, nbytes, hipMemcpyDeviceToDevice, (hipStream_t)stream), "memcpy dtod");
    return UQ_OK;
}

uq_status uq_stream_synchronize(void *stream) {
    UQ_HIP(hipStreamSynchronize((hipStream_t)stream), "stream synchronize");
    return UQ_OK;
}

}  // extern "C"
