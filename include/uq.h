/*
 * uq.h -- C ABI of the MI355X quantized linear-layer library (libuq.so).
 *
 * Drop-in boundary for unltd-tensor's quantized-matmul operator API
 * (crates/unltd-tensor/src/lib.rs:128-131 re-exports, quants.rs bodies).
 * Every entry point below cites the reference function it replaces.
 *
 * Conventions
 *  - Weights are GGUF tensors: [dim_out] rows, each row dim_in weights packed
 *    in blocks of the row's dtype, row-major, block bytes unchanged
 *    (quants.rs:414-421). dtype values are ggml type ids (min_forward.rs:39-48).
 *  - The reference panics on bad arguments (assert_eq!/panic!); here every
 *    panic class is a uq_status code, and uq_last_error() returns the
 *    message of the calling thread's last failure. No entry point aborts.
 *  - Host-pointer entry points (uq_gemv_quant, ...) take the reference's
 *    slices as (pointer, length) pairs, copy to the current HIP device, run,
 *    and copy back. They are reentrant (thread-safe, one HIP stream per
 *    calling thread).
 *  - Device entry points take device pointers and a hipStream_t (void*; NULL
 *    = the null stream). They are asynchronous on that stream and allocate
 *    no device memory, except uq_gemm and uq_gemm_q8k (see there). Weights live behind a
 *    uq_weights handle whose bytes are copied to HBM unchanged.
 *  - Numerics: uq_gemv_quant / uq_gemv / uq_gemm / uq_ffn_swiglu follow
 *    gemv_quant's semantics (f32 result of the exact dequantized weights times
 *    f32 x; matched within |y-r| <= 1e-4 + 1e-3*|r|). uq_gemv_quant_q8k /
 *    uq_gemv_q8k / uq_gemm_q8k, uq_quantize_q8_k, the dequantize and unpack
 *    exports are bit-exact with the reference.
 */
#ifndef UQ_H
#define UQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids, DType mapping of dtype_of (min_forward.rs:39-48). */
typedef enum uq_dtype {
    UQ_F32 = 0,
    UQ_F16 = 1, /* recognised, no dot kernel (gemv_quant panics, quants.rs:446) */
    UQ_Q8_0 = 8,
    UQ_Q4_K = 12,
    UQ_Q6_K = 14
} uq_dtype;

typedef enum uq_status {
    UQ_OK = 0,
    UQ_ERR_LEN = 1,            /* assert_eq!(len ...): quants.rs:430-452, :482-505, :535-539 */
    UQ_ERR_BLOCK_MULTIPLE = 2, /* dim_in % 256 != 0: quants.rs:435-439 (min_forward.rs:55-66) */
    UQ_ERR_DTYPE = 3,          /* unsupported dtype panic: quants.rs:446, :497-499 */
    UQ_ERR_ARG = 4,            /* null pointer, bad handle, size out of range */
    UQ_ERR_HIP = 5,            /* HIP runtime failure (message in uq_last_error) */
    UQ_ERR_NO_DEVICE = 6,      /* no usable gfx950 device */
    UQ_ERR_TOKEN = 7,          /* token id >= vocab: LoadError::corrupt of embed, min_forward.rs:168-173 */
    /* GGUF loader (uq_gguf.h); LoadError variants of unltd-core/src/lib.rs:19-96 */
    UQ_ERR_FILE = 8,           /* BadFile: corrupt or truncated file */
    UQ_ERR_MAGIC = 9,          /* BadMagic */
    UQ_ERR_VERSION = 10,       /* UnsupportedVersion */
    UQ_ERR_TENSOR_BOUNDS = 11, /* TensorOutOfBounds */
    UQ_ERR_TENSOR_OVERLAP = 12,/* TensorOverlap */
    UQ_ERR_TENSOR_ALIGN = 13,  /* MisalignedTensor */
    UQ_ERR_GGML_TYPE = 14,     /* UnknownGgmlType */
    UQ_ERR_MISSING_TENSOR = 15,/* MissingTensor */
    UQ_ERR_ELEMENT_COUNT = 16, /* ElementCount */
    UQ_ERR_IO = 17             /* Io */
} uq_status;

/* Q8_K activation block, quants.rs:235-242 ({f32 d; i8 qs[256]; i32 bsums[16]}). */
typedef struct uq_q8k_block {
    float d;
    int8_t qs[256];
    int32_t bsums[16];
} uq_q8k_block;

/* Message of the calling thread's last failing call ("" if none). */
const char *uq_last_error(void);
/* Static name of a status code. */
const char *uq_status_name(uq_status s);
/* Bytes of one row of dim_in weights (min_forward.rs:52-80); 0 if refused. */
size_t uq_row_bytes(uq_dtype dtype, size_t dim_in);

/* ===================== host-pointer mirrors of unltd-tensor ============== */

/* gemv_quant (quants.rs:422-466): out[j] = (f32) dot(x[..dim_in], row_j).
 * F32, Q4_K, Q6_K as the reference; Q8_0 accepted (GGUF closed form) where
 * the reference panics. x_len >= dim_in (x may be longer, :431). */
uq_status uq_gemv_quant(float *out, size_t out_len, const float *x, size_t x_len,
                        const uint8_t *w, size_t w_len, size_t dim_in,
                        size_t dim_out, uq_dtype dtype);

/* gemv_quant_q8k (quants.rs:474-515): x quantized to Q8_K once, each row dotted
 * with dot_q4_k_q8_k / dot_q6_k_q8_k. Q4_K and Q6_K only. Bit-exact. */
uq_status uq_gemv_quant_q8k(float *out, size_t out_len, const float *x,
                            size_t x_len, const uint8_t *w, size_t w_len,
                            size_t dim_in, size_t dim_out, uq_dtype dtype);

/* quantize_q8_k (quants.rs:250-290): x_len % 256 == 0, out_blocks == x_len/256. */
uq_status uq_quantize_q8_k(uq_q8k_block *out, size_t out_blocks, const float *x,
                           size_t x_len);

/* dequantize_q4_k (quants.rs:534-567): w_len == out_len/256*144, bit-exact. */
uq_status uq_dequantize_q4_k(float *out, size_t out_len, const uint8_t *w,
                             size_t w_len);
/* Q6_K to f32: w = d*(sc*q), the exact product dot_q6_k forms (quants.rs:195);
 * no reference function exists, bit-exact with that product. */
uq_status uq_dequantize_q6_k(float *out, size_t out_len, const uint8_t *w,
                             size_t w_len);
/* Q8_0 to f32: w = d*q (GGUF closed form; no reference kernel). */
uq_status uq_dequantize_q8_0(float *out, size_t out_len, const uint8_t *w,
                             size_t w_len);

/* Integer unpack of the element maps (quants.rs:146-151 for Q4_K, :185-194 for
 * Q6_K): per block 256 quants (Q4_K nibble 0..15; Q6_K raw 6-bit 0..63, the
 * reference's q is raw-32), the per-group scales and the f32 block scales
 * (f16_to_f32, quants.rs:44-72). Debug exports for bit-exact checks. */
uq_status uq_unpack_q4_k(const uint8_t *w, size_t nblocks, uint8_t *q,
                         uint8_t *sc, uint8_t *m, float *d, float *dmin);
uq_status uq_unpack_q6_k(const uint8_t *w, size_t nblocks, uint8_t *q,
                         int8_t *sc, float *d);
uq_status uq_unpack_q8_0(const uint8_t *w, size_t nblocks, int8_t *q, float *d);

/* f16_to_f32 (quants.rs:44-72) over an array, on the device; bit-exact
 * including the reference's quiet-NaN canonicalisation. */
uq_status uq_f16_to_f32(float *out, const uint16_t *h, size_t n);

/* swiglu (kernels.rs:174-182): out = (g/(1+expf(-g)))*u, f32. */
uq_status uq_swiglu(float *out, const float *gate, const float *up, size_t n);

/* ========================= device-resident API ========================== */

typedef struct uq_weights_s *uq_weights;

/* Copy one GGUF tensor's bytes to HBM unchanged. nbytes must equal
 * uq_row_bytes(dtype, dim_in) * dim_out (checked like gemv_quant, :448-452).
 * Uploads to the current HIP device. */
uq_status uq_weights_upload(uq_weights *out, const void *bytes, size_t nbytes,
                            uq_dtype dtype, size_t dim_in, size_t dim_out);
uq_status uq_weights_free(uq_weights w);
/* Shape of a handle (any pointer may be NULL). */
uq_status uq_weights_info(uq_weights w, uq_dtype *dtype, size_t *dim_in,
                          size_t *dim_out, size_t *nbytes);

/* d_y[dim_out] = W . d_x[dim_in] with gemv_quant semantics (quants.rs:422-466). */
uq_status uq_gemv(uq_weights w, const float *d_x, float *d_y, void *stream);

/* Several projections of one activation vector in one launch:
 * d_y[i] = W[i] . d_x for i < count (count <= UQ_GEMV_BATCH_MAX), e.g. the
 * q, k and v projections of a token. All W[i] share dtype and dim_in.
 * gemv_quant semantics; every d_y[i] equals what uq_gemv(W[i]) writes, bit
 * for bit. No reference counterpart (the reference calls gemv_quant_q8k once
 * per projection, qwen35_forward.rs:365-401); it saves the per-launch
 * activation preparation of the small projections. */
#define UQ_GEMV_BATCH_MAX 8
uq_status uq_gemv_batch(const uq_weights *w, float *const *d_y, size_t count,
                        const float *d_x, void *stream);

/* d_y = gemv_quant_q8k(W, d_x) (quants.rs:474-515), bit-exact. */
uq_status uq_gemv_q8k(uq_weights w, const float *d_x, float *d_y, void *stream);

/* uq_gemv_batch with gemv_quant_q8k semantics (Q4_K / Q6_K): every d_y[i]
 * equals gemv_quant_q8k(W[i], d_x) bit for bit. No reference counterpart
 * (one gemv_quant_q8k call per projection, qwen35_forward.rs:365-401). */
uq_status uq_gemv_q8k_batch(const uq_weights *w, float *const *d_y, size_t count,
                            const float *d_x, void *stream);

/* Batched prefill: d_y[m][dim_out] = W . d_x[m][dim_in] for m < m_rows, with
 * gemv_quant semantics per row (the reference feeds prefill tokens one at a
 * time, greedy.rs:55-65; each row equals gemv_quant of that token).
 * Q4_K, Q6_K and Q8_0 with m_rows >= 2 and dim_in a multiple of 256 (tensor
 * below 4 GiB, activation planes below 2 GiB) run on the f16 MFMA, one weight
 * pass per 32-128-row tile; the row results are within the gemv_quant
 * tolerance plus 2^-22 * sum_e |x_e w_e| (the matrix cores' f32
 * accumulation within each 256-k block; when K is split across workgroups
 * the partial tiles stay f64 and are summed in range order, adding no
 * term). m_rows == 1 and other shapes run as m_rows GEMVs. A NaN or
 * infinity in a row of d_x makes that row of d_y NaN. The MFMA path uses a
 * library-owned device workspace per (device, stream) of about
 * 4*m_rows*dim_in bytes (plus f64 split-K partial tiles, 8 bytes per output
 * and K range, when the output tiles do not cover the CUs), allocated on
 * first use and grown when a call
 * needs more; a grown-out buffer is kept, never freed, so work queued on the
 * stream or a graph captured earlier stays valid. A call can be captured in
 * a HIP graph once a call of that size or larger has run on the stream. */
uq_status uq_gemm(uq_weights w, size_t m_rows, const float *d_x, float *d_y,
                  void *stream);

/* Batched prefill in the reference forward's numerics: d_y[m][dim_out] =
 * gemv_quant_q8k(W, d_x[m][dim_in]) (quants.rs:474-515) for m < m_rows, bit
 * for bit per row. The reference prefills one token at a time through
 * gemv_quant_q8k (greedy.rs:55-65; qwen35_forward.rs:365-401); this is
 * those m_rows calls in one weight pass: each row quantized to Q8_K as
 * quantize_q8_k does, the eight integer lane sums per block formed exactly
 * on the f16 MFMA, the f32 epilogue of dot_q4_k_q8_k / dot_q6_k_q8_k
 * replayed per output in the reference's order. Q4_K and Q6_K only
 * (UQ_ERR_DTYPE otherwise, as the reference panics, quants.rs:497-499);
 * m_rows == 1 runs uq_gemv_q8k. Workspace (about 2*m_rows*dim_in bytes) as
 * uq_gemm's: library-owned per (device, stream), grown on demand, never
 * freed; a call can be captured in a HIP graph once one of that size or
 * larger has run on the stream. */
uq_status uq_gemm_q8k(uq_weights w, size_t m_rows, const float *d_x, float *d_y,
                      void *stream);

/* uq_gemm_q8k of several weights over the same rows in one launch: d_y[i] =
 * uq_gemm_q8k(W[i], m_rows, d_x) bit for bit, for i < count (count <=
 * UQ_GEMM_Q8K_BATCH_MAX), e.g. the qkv, gate, beta and alpha projections of
 * a GatedDeltaNet layer's tokens. All W[i] share dtype (Q4_K or Q6_K) and
 * dim_in; each d_y[i] is [m_rows][dim_out of W[i]]. The rows are quantized
 * once and one grid covers every weight's column tiles (above 128 rows the
 * weights under 128 columns run in a second grid). No reference
 * counterpart (one gemv_quant_q8k call per projection and token,
 * qwen35_forward.rs:365-401, greedy.rs:55-65). Workspace as uq_gemm_q8k's.
 * m_rows == 1 runs uq_gemv_q8k_batch. */
#define UQ_GEMM_Q8K_BATCH_MAX 4
uq_status uq_gemm_q8k_batch(const uq_weights *w, float *const *d_y, size_t count,
                            size_t m_rows, const float *d_x, void *stream);

/* uq_gemm that allocates nothing: no reference counterpart. For callers that
 * cannot allocate device memory inside the call (HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same arguments, kernels
 * and results as uq_gemm (the same bits); the workspace is a fixed device array
 * of UQ_GEMM_SCRATCH_BYTES inside the library, one per GPU, held until the
 * process ends. A call whose workspace would not fit (roughly
 * 4*m_rows*dim_in bytes, plus 8 bytes per output and K range when K is
 * split)
 * fails with UQ_ERR_ARG and launches nothing. Calls on one GPU share the
 * array: calls that may overlap on a GPU (other streams, other threads)
 * race and must be ordered by the caller. */
#define UQ_GEMM_SCRATCH_BYTES (64u << 20)
uq_status uq_gemm_static(uq_weights w, size_t m_rows, const float *d_x, float *d_y,
                         void *stream);

/* Gated FFN of one token (qwen35_forward.rs:713-768): d_h = swiglu(gate.x, up.x)
 * (kernels.rs:174-182) computed in the GEMV epilogue, then d_y = down.d_h.
 * gate/up: [n_ff][n]; down: [n][n_ff]. d_h holds n_ff floats. */
uq_status uq_ffn_swiglu(uq_weights gate, uq_weights up, uq_weights down,
                        const float *d_x, float *d_h, float *d_y, void *stream);

/* The reference FFN (qwen35_forward.rs:735-765) on the device: d_g =
 * gemv_quant_q8k(gate, d_x), d_u = gemv_quant_q8k(up, d_x) (one launch),
 * d_h = swiglu(d_g, d_u) (kernels.rs:174-182), d_y = gemv_quant_q8k(down,
 * d_h). d_g, d_u and d_y (given d_h) are bit-exact; d_h is within 2 ulp of
 * the reference's swiglu, whose expf is the platform libm's (here expf is
 * evaluated in f64 and rounded once). gate/up: [n_ff][n]; down: [n][n_ff];
 * Q4_K or Q6_K. d_g, d_u, d_h hold n_ff floats (the reference's g, u, sw). */
uq_status uq_ffn_swiglu_q8k(uq_weights gate, uq_weights up, uq_weights down,
                            const float *d_x, float *d_g, float *d_u, float *d_h,
                            float *d_y, void *stream);

/* swiglu (kernels.rs:174-182) on device arrays: d_out = (g/(1+expf(-g)))*u. */
uq_status uq_swiglu_d(float *d_out, const float *d_gate, const float *d_up, size_t n,
                      void *stream);

/* Device f32 dequantization of a whole handle into d_out[dim_out*dim_in]
 * (dequantize_q4_k semantics, bit-exact; Q6_K/Q8_0 closed forms). */
uq_status uq_dequantize(uq_weights w, float *d_out, void *stream);

/* Embedding lookup, embed (min_forward.rs:160-184): for r < n_tokens,
 * d_out[r*dim_in .. (r+1)*dim_in) = row tokens[r] of w, copied (F32) or
 * dequantized bit-exactly as dequantize_q4_k (Q4_K). Q6_K / Q8_0 rows use
 * the closed forms of uq_dequantize_q6_k / _q8_0 (the reference refuses them
 * when it opens the model). tokens is a HOST array: every id is checked
 * against w's dim_out (the vocabulary) before any launch, and the first id
 * out of range fails with UQ_ERR_TOKEN, as the reference returns an error
 * rather than clamping. The ids travel in the kernel arguments (256 per
 * launch), so the call allocates nothing. n_tokens == 0 is a no-op. */
uq_status uq_embed(uq_weights w, const uint32_t *tokens, size_t n_tokens, float *d_out, void *stream);

/* ------------------------------------------------------------------------
 * Device memory and stream plumbing for callers without their own HIP
 * binding (the Rust FFI crate, the ctypes tests). Thin wrappers over the
 * HIP runtime of the current device.
 * --------------------------------------------------------------------- */
uq_status uq_device_count(int *n);
uq_status uq_device_name(char *buf, size_t len);
uq_status uq_malloc(void **d_ptr, size_t nbytes);
uq_status uq_free(void *d_ptr);
uq_status uq_memcpy_htod(void *d_dst, const void *src, size_t nbytes, void *stream);
uq_status uq_memcpy_dtoh(void *dst, const void *d_src, size_t nbytes, void *stream);
uq_status uq_memcpy_dtod(void *d_dst, const void *d_src, size_t nbytes, void *stream);
uq_status uq_stream_synchronize(void *stream);

#ifdef __cplusplus
}
#endif
#endif /* UQ_H */
