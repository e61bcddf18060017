/*
 * tomoul_hip.h -- C ABI of the MI355X (gfx950) matrix-multiply backend.
 *
 * A drop-in for the backends behind Tomoul's ops.matmul / ops.matmulBias /
 * ops.matmulParallel / ops.matvec and quantization.matmulF32Q8Simd /
 * matmulF32Q8KSimd / matmulF32Q4Simd.  Every pointer argument of the
 * "host" entry points is a plain host pointer, exactly as the Zig call sites
 * pass slices today; the "_dev" entry points take device pointers that are
 * already resident in HBM plus a hipStream_t (passed as void*).
 *
 * Matrices are row-major: A is [M,K] (lda = K), B is [K,N] (ldb = N) -- the
 * [in, out] layout every reference caller hands over -- and C is [M,N]
 * (ldc = N).  Quantized B uses the reference's in-memory layouts unchanged:
 *   Q8_0  int8  q[K*N] + one f32 scale            (quantization.zig:39-90)
 *   Q8_K  int8  q[K*N] + f32 scales[ceil(K*N/32)],
 *         scale of element (k,j) = scales[(k*N+j)/block]
 *                                                 (quantization.zig:327-403)
 *   Q4_0  uint8 packed[ceil(K*N/2)] + one f32 scale; element e is the low
 *         nibble of byte e/2 when e is even, the high nibble when odd, read
 *         as a two's-complement 4-bit value   (quantization.zig:627-717)
 * The format ids equal the .tl header's quant-format byte
 * (src/core/loader.zig:23-29).
 *
 * Return value: 0 on success, a negative TML_ERR_* code otherwise; the
 * message of the last failure on the calling thread is available from
 * tml_hip_last_error().  Sizes are int64_t; a negative size is
 * TML_ERR_INVALID_SHAPE, M == 0 or N == 0 is a successful no-op.
 *
 * Threading: calls are thread-compatible, not thread-safe (as the reference's
 * callers: one model-forward thread, src/core/ops.zig:485).  All calls on
 * one device share that device's split-K workspace, so "_dev" calls issued
 * concurrently on different streams of the same device race; issue them on
 * one stream.
 */
#ifndef TOMOUL_HIP_H
#define TOMOUL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  The first three mirror the reference's OpsError /
 * QuantError members (src/core/ops.zig:47-52, quantization.zig:25-30). */
#define TML_OK 0
#define TML_ERR_INVALID_SHAPE (-1)  /* OpsError.InvalidShape                  */
#define TML_ERR_SHAPE_MISMATCH (-2) /* OpsError.ShapeMismatch                 */
#define TML_ERR_OUT_OF_MEMORY (-3)  /* OpsError.OutOfMemory (device memory)   */
#define TML_ERR_INVALID_FORMAT (-4) /* QuantError.InvalidFormat               */
#define TML_ERR_INVALID_ARG (-5)    /* null pointer, bad block size, ...      */
#define TML_ERR_NO_DEVICE (-6)      /* no usable HIP device                   */
#define TML_ERR_HIP (-7)            /* a HIP runtime call failed              */
/* .tl files: the reference's LoadError members (src/core/loader.zig:11-20). */
#define TML_ERR_INVALID_MAGIC (-8)            /* LoadError.InvalidMagic           */
#define TML_ERR_UNSUPPORTED_VERSION (-9)      /* LoadError.UnsupportedVersion     */
#define TML_ERR_CORRUPTED_FILE (-10)          /* LoadError.CorruptedFile          */
#define TML_ERR_TENSOR_NOT_FOUND (-11)        /* LoadError.TensorNotFound         */
#define TML_ERR_FILE_NOT_FOUND (-12)          /* LoadError.FileNotFound           */
#define TML_ERR_UNSUPPORTED_QUANT_FORMAT (-13) /* LoadError.UnsupportedQuantFormat */

/* Weight formats (= .tl quant-format byte, src/core/loader.zig:23-29). */
#define TML_FMT_F32 0
#define TML_FMT_Q8_0 1
#define TML_FMT_Q4_0 2
#define TML_FMT_Q8_K 3
#define TML_FMT_F16 4  /* IEEE binary16 [K,N], F16Tensor / matmulF32F16
                          (src/core/quantization.zig:1859-1962); .tl code 4 */
/* Per-output-column scales: an extension, not a reference format (the
 * reference quantizes per tensor, Q8_0 / Q4_0, or per 32 elements, Q8_K).
 * Data exactly as Q8_0 / Q4_0; `scales` holds N floats, scale of column n =
 * scales[n]; the per-tensor `scale` argument is ignored.  Column n is
 * quantized by the per-tensor quantizer applied to that column alone
 * (tml_hip_quantize_cols).  For weights quantized "symmetric int8 with a
 * per-output-row fp32 scale" ([out,in] row = [in,out] column). */
#define TML_FMT_Q8_0_PC 17
#define TML_FMT_Q4_0_PC 18

/* Activation applied after the bias, in the kernel epilogue. */
#define TML_ACT_NONE 0
#define TML_ACT_GELU_ERF 1  /* ops.geluExact: x/2 (1 + erf(x/sqrt 2)), erf by Abramowitz-Stegun
                               7.1.26 as in src/core/ops.zig:2000-2057 */
#define TML_ACT_GELU_TANH 2 /* ops.gelu: x/2 (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3))), tanh by the
                               reference's Pade approximant on its 8-wide vector part and exact
                               tanh on the flat tail of (M*N) % 8 elements, src/core/ops.zig:1947-1998 */

/* ---------------------------------------------------------------- setup */

/* Selects the current HIP device and creates the library's stream.  Called
 * implicitly by every entry point; calling it first surfaces device errors
 * early.  No counterpart in the reference (zblas needs no init). */
int tml_hip_init(void);

/* Frees every device buffer, registered weight and stream of the library. */
void tml_hip_shutdown(void);

/* Message for the last failing call on this thread ("" if none). */
const char *tml_hip_last_error(void);

/* Writes the device name (e.g. "AMD Instinct MI355X") into buf. */
int tml_hip_device_name(char *buf, size_t len);

/* ---------------------------------------------------- host-pointer API
 * Blocking.  Operands and C pass through the device's pinned staging
 * buffers (up to 256 MiB a direction; larger ones are sent from the
 * caller's memory), with host copies on up to seven worker threads the
 * library starts on first use and joins at process exit. */

/* C = alpha * A.B + beta * C.  Replaces zblas.sgemm(m, n, k, a, b, c, alpha,
 * beta) at src/core/ops.zig:273 and :513, and blas.sgemm -> cblas_sgemm
 * (RowMajor, NoTrans, NoTrans, lda=K, ldb=N, ldc=N) at src/core/blas.zig:68-94
 * (call sites src/core/ops.zig:269, :448, :516).  With beta == 0 the input
 * contents of C are ignored (BLAS convention). */
int tml_hip_sgemm(int64_t M, int64_t N, int64_t K, const float *A, const float *B, float *C, float alpha,
                  float beta);

/* C = A.B + bias[N] broadcast over rows.  Replaces zblas.sgemmBias(m, n, k,
 * a, b, bias.ptr, c) at src/core/ops.zig:442 (ops.matmulBias,
 * src/core/ops.zig:422-471). */
int tml_hip_sgemm_bias(int64_t M, int64_t N, int64_t K, const float *A, const float *B, const float *bias,
                       float *C);

/* y[M] = alpha * A[M,N].x[N] + beta * y.  Replaces zblas.sgemv(m, n, a, x,
 * y, alpha, beta) at src/core/ops.zig:630 (ops.matvec, :611-642). */
int tml_hip_sgemv(int64_t M, int64_t N, const float *A, const float *x, float *y, float alpha, float beta);

/* C = A . dequant(Q8_0 B).  Replaces zblas.sgemmQ8(m, n, k, a, b.data,
 * scale, c) at src/core/quantization.zig:236 (matmulF32Q8Simd, :207-314). */
int tml_hip_sgemm_q8(int64_t M, int64_t N, int64_t K, const float *A, const int8_t *Bq, float scale, float *C);
/* Arithmetic of the Q8_0 / Q4_0 products (every entry point and format,
 * per-column forms included): past the decoder rows (M > 8; K a multiple of
 * 8, even N), and on a prepared weight at the M = 2-8 calls the matrix-core
 * GEMV takes, they run on the bf16 matrix cores, the int weights exact in
 * bf16 and each fp32 activation split into two bf16 terms
 * (|x - hi - lo| <= 2^-17 |x|), accumulated in fp32; otherwise on fp32
 * multiply-adds.  Both agree with
 * the reference's dequantize-then-fp32-accumulate result to ~1e-5 relative;
 * infinities and NaNs in A give what the reference gives.  Limit: the
 * per-tensor scale multiplies the finished sum (the reference multiplies
 * each element, a * (q * s)), so finite activations large enough that
 * x * q overflows fp32 (|x| > FLT_MAX / 127 for int8, / 8 for int4) give
 * inf or NaN where the reference stays finite.  On the matrix cores hi is
 * taken from x clamped to the largest finite bf16, so a finite x near
 * FLT_MAX keeps a finite product where q is 0 or +-1. */

/* C = A . dequant(Q8_K B).  Replaces zblas.sgemmQ8K(m, n, k, a, b.data,
 * b.scales, b.block_size, c) at src/core/quantization.zig:555
 * (matmulF32Q8KSimd, :528-617).  scales holds ceil(K*N/block) values;
 * block must be positive (the reference always uses 32). */
int tml_hip_sgemm_q8k(int64_t M, int64_t N, int64_t K, const float *A, const int8_t *Bq, const float *scales,
                      int64_t block, float *C);

/* C = A . dequant(Q4_0 B), Bp holding ceil(K*N/2) packed bytes.  Replaces
 * the in-tree loop of matmulF32Q4Simd (src/core/quantization.zig:829-957);
 * the reference has no zblas entry for Q4_0.  Unlike the reference's 32-wide
 * SIMD loop, odd N is handled exactly (every element is addressed as
 * k*N + j). */
int tml_hip_sgemm_q4(int64_t M, int64_t N, int64_t K, const float *A, const uint8_t *Bp, float scale, float *C);

/* C[M,N] = A[M,K] . f32(Bh[K,N]) with Bh binary16: zblas.sgemmF16 at
 * src/core/quantization.zig:1946 (matmulF32F16, :1921-1962; its fallback
 * accumulates a * f32(b) in f32, ascending k). */
int tml_hip_sgemm_f16(int64_t M, int64_t N, int64_t K, const float *A, const uint16_t *Bh, float *C);

/* Generic host-pointer matmul with an optional fused bias:
 *   C = A . dequant(B) + bias      (bias may be NULL)
 * fmt/scale/scales/block as for tml_hip_gemm_dev below.  Replaces the
 * quantized branch of matmulWithWeightBias (src/core/attention.zig:132-149,
 * duplicated at src/core/transformer.zig:147-166), which runs the weight-only
 * matmul and then a separate addBiasInPlace pass; here the bias is applied in
 * the kernel epilogue. */
int tml_hip_gemm(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B, float scale,
                 const float *scales, int64_t block, const float *bias, float *C);

/* tml_hip_gemm with an activation fused after the bias:
 *   C = act(A . dequant(B) + bias)
 * Replaces the Whisper FFN's fc1 (src/models/whisper/encoder.zig:244-247 and
 * decoder.zig:336-338: matmul, addBiasInPlace, geluExact) and the transformer
 * FFN's first linear (src/core/transformer.zig:218-221: matmulWithWeightBias,
 * then ops.gelu) with one launch. */
int tml_hip_gemm_act(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B, float scale,
                     const float *scales, int64_t block, const float *bias, int act, float *C);

/* tml_hip_gemm with the residual connection fused after the bias:
 *   C = (A . dequant(B) + bias) + residual      (residual: M*N floats)
 * Replaces the FFN / attention down-projection followed by its residual
 * add: matmulWithWeightBias then ops.addInPlace (src/core/transformer.zig:
 * 223-228), and Whisper's matmul, addBiasInPlace, ops.add
 * (src/models/whisper/encoder.zig:249-253).  Same additions in the same
 * order as the reference, so the result is the separate passes' result. */
int tml_hip_gemm_residual(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B, float scale,
                          const float *scales, int64_t block, const float *bias, const float *residual, float *C);

/* Host-pointer form of tml_hip_quantize_dev below (synchronous): the GPU
 * replacement for the load-time quantizers quantizeQ8 / quantizeQ8K /
 * quantizeQ4 (src/core/quantization.zig:98-129, :406-446, :721-754) that
 * produce the in-memory layouts consumed above. */
int tml_hip_quantize(int fmt, int64_t n, const float *w, void *q, float *scales);

/* Weight residency.  Weights are immutable after load in the reference
 * (AttentionWeights / TransformerBlockWeights own them until deinit,
 * src/core/attention.zig:54-86), so a host buffer registered here is copied
 * to HBM once; later host-pointer calls whose B (or Q8_K scales) pointer and
 * size match a registered buffer use the resident copy instead of uploading
 * it again.  Registering an already registered pointer refreshes the copy.
 * No counterpart in the reference. */
int tml_hip_weight_register(const void *host, size_t bytes);
int tml_hip_weight_release(const void *host);

/* ------------------------------------------------------ device-pointer API */

/* The compute entry point behind every call above, on resident operands:
 *   C = alpha * (A . dequant(B)) + beta * C + bias
 * fmt       TML_FMT_*; B points at the f32 / int8 / packed-int4 data.
 * scale     per-tensor scale of Q8_0 / Q4_0 (ignored for F32 and Q8_K).
 * scales    device pointer to the Q8_K block scales (NULL otherwise).
 * block     Q8_K block size (ignored otherwise).
 * bias      device pointer to N floats, or NULL.
 * stream    hipStream_t to launch on (NULL = the null stream).
 * All pointers are device pointers.  Asynchronous: returns after the launch.
 * B may have any alignment.  At M <= 8 the GEMV reads B in 4- to 16-byte
 * chunks when B is 4-byte aligned (also when N is not a whole number of
 * chunks), and element by element otherwise, which is several times slower.
 *
 * Workspace and HIP graphs: a problem whose plan splits K uses the device's
 * split-K workspace, which the library grows (hipMalloc) the first time a
 * call needs more than earlier calls did.  Growth is refused with
 * TML_ERR_INVALID_ARG while `stream` is being captured, so run every call
 * once eagerly before capturing it.  A grown workspace never frees the old
 * one before tml_hip_shutdown: a graph captured earlier stays valid however
 * the workspace grows afterwards. */
int tml_hip_gemm_dev(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B, float scale,
                     const float *scales, int64_t block, const float *bias, float *C, float alpha, float beta,
                     void *stream);

/* tml_hip_gemm_dev with the full fused epilogue:
 *   C = act((alpha * (A . dequant(B)) + beta * C + bias) + residual)
 * residual: device pointer to M*N floats or NULL; it is read before C is
 * written, element by element, so it may equal C.  act: TML_ACT_*.  The
 * device-pointer form of tml_hip_gemm_act / tml_hip_gemm_residual. */
int tml_hip_gemm_ex_dev(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B, float scale,
                        const float *scales, int64_t block, const float *bias, const float *residual, int act,
                        float *C, float alpha, float beta, void *stream);

/* Allocation-free form of tml_hip_gemm_ex_dev.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory -- code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  Same arguments, same kernels and plans, same results bit for
 * bit; the split-K scratch (partial sums, arrival counters and the zero
 * block the kernels read out-of-range lanes from) is a static device array of
 * TML_NOALLOC_SCRATCH_BYTES per GPU, held from the library's load until the
 * process ends, instead of the library's growable workspace.  The call makes
 * no hipMalloc / hipFree.  Set-up -- looking up this GPU's address of the
 * array and clearing its counters -- happens in tml_hip_init (or on the first
 * call on a device, which must then not be under stream capture).
 * A problem whose plan needs more scratch than the array holds is refused
 * with TML_ERR_INVALID_SHAPE before any launch.  All calls on one GPU share
 * its array: calls that overlap on one GPU (several streams, several host
 * threads) race; issue them on one stream. */
#define TML_NOALLOC_SCRATCH_BYTES (16u << 20)
int tml_hip_gemm_ex_dev_noalloc(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B, float scale,
                                const float *scales, int64_t block, const float *bias, const float *residual, int act,
                                float *C, float alpha, float beta, void *stream);

/* On-device quantizers, bit-identical to the reference's Zig quantizers
 * (quantizeQ8 quantization.zig:98-129, quantizeQ8K :406-446, quantizeQ4
 * :721-754) and its f32 -> f16 converter toF16 (:1907-1917, IEEE round to
 * nearest even).  w holds n floats; q receives n int8 (Q8_0 / Q8_K),
 * ceil(n/2) packed bytes (Q4_0) or n binary16 values (F16); scales receives
 * 1 float (Q8_0 / Q4_0), ceil(n/32) floats (Q8_K) or nothing (F16, may be
 * NULL).  Device pointers, asynchronous on stream. */
int tml_hip_quantize_dev(int fmt, int64_t n, const float *w, void *q, float *scales, void *stream);

/* Read floor of the decoder GEMVs.  No counterpart in the reference: a
 * measurement aid for callers and benchmarks that want to know what one
 * launch streaming `bytes` of device memory costs on this GPU.  Reads
 * bytes (0 <= bytes < 2^31) at src with 16-byte loads, chunks_per_lane
 * (1, 2, 4 or 8) of them per lane, all issued before any is used, and
 * writes one value per workgroup -- ceil(bytes / (chunks_per_lane * 4096))
 * floats -- to out.  Asynchronous on stream. */
int tml_hip_stream_read_dev(const void *src, int64_t bytes, int chunks_per_lane, float *out, void *stream);

/* Per-output-column quantizers for TML_FMT_Q8_0_PC / TML_FMT_Q4_0_PC: w is
 * W[K,N] row-major; q receives the Q8_0 / Q4_0 data of W, scales the N
 * column scales.  No counterpart in the reference (see TML_FMT_Q8_0_PC).
 * _dev: device pointers, asynchronous; the other: host pointers, blocking. */
int tml_hip_quantize_cols_dev(int fmt, int64_t K, int64_t N, const float *w, void *q, float *scales, void *stream);
int tml_hip_quantize_cols(int fmt, int64_t K, int64_t N, const float *w, void *q, float *scales);

/* ------------------------------------------------------ prepared weights */

/* Device-native copy of an immutable weight for decoder products.  The
 * reference's weights are immutable after load and owned by
 * AttentionWeights / TransformerBlockWeights until deinit
 * (src/core/attention.zig:54-86, src/core/transformer.zig:31-68), so a
 * backend may keep them in whatever layout its kernels read best.  The
 * prepared copy stores column n of B as row n, zero padded to a multiple of
 * 16 bytes, its k in an order interleaved across 16-byte chunks so that
 * the lanes reading consecutive chunks read contiguous activations (plain K
 * order for f32); a GEMV then reads each output's weights as one contiguous
 * run and needs no cross-workgroup reduction (M <= 8, every format; Q4_0
 * above M = 4 runs on the [K,N] weight, measured faster there).  No
 * counterpart in the reference (its CPU loops read B in place).
 *
 * tml_hip_prepare_dev: fmt is TML_FMT_F32, TML_FMT_F16, TML_FMT_Q8_0 or
 *   TML_FMT_Q4_0;
 *   B is the device [K,N] weight in the layouts above, scale the Q8_0 /
 *   Q4_0 per-tensor scale.  The copy is built asynchronously on `stream`.
 *   B must stay valid and unchanged while the handle is used: calls with
 *   more rows than the prepared kernel covers run on B itself.
 * tml_hip_gemm_prepared: C = alpha * A[M,K] . dequant(B) + beta * C + bias
 *   (bias may be NULL), device pointers, asynchronous on `stream`.
 * tml_hip_prepared_free: waits for the device, then frees the copy.
 *
 * Host-pointer calls with a registered weight (tml_hip_weight_register) at
 * those row counts build and use such a copy automatically. */
typedef struct tml_prepared_weight *tml_prepared_t;
int tml_hip_prepare_dev(int fmt, int64_t K, int64_t N, const void *B, float scale, void *stream,
                        tml_prepared_t *out);
/* tml_hip_prepare_dev for every preparable format, per-channel ones
 * included: `scales` is the device pointer to their N column scales (copied
 * into the handle), NULL for the other formats. */
int tml_hip_prepare_ex_dev(int fmt, int64_t K, int64_t N, const void *B, float scale, const float *scales,
                           void *stream, tml_prepared_t *out);
int tml_hip_gemm_prepared(tml_prepared_t w, int64_t M, const float *A, const float *bias, float *C, float alpha,
                          float beta, void *stream);

/* A prepared weight from a matrix stored as N rows of K elements, i.e. B
 * transposed: W row n (at W + n * ldw bytes) is column n of B.  This is the
 * layout of the tied vocabulary projection, logits = x . token_embedding^T
 * with token_embedding [n_vocab, d] (src/models/whisper/decoder.zig:
 * 936-940, :377-383, :619-622), which the reference transposes on every
 * decode step; here the embedding is used as it is stored.  It is also the
 * PyTorch [out,in] layout of weights exported untransposed.
 * fmt F32, F16, Q8_0 (one int8 per element) or Q4_0 (two per byte, even k
 * low; K must be even so each row starts a byte).  F32 rows that are a
 * multiple of 16 bytes, with W and ldw 16-byte aligned, are used in place
 * (no copy; W must stay valid and unchanged while the handle lives);
 * otherwise the prepared layout is built on `stream` in a new buffer.  Products with more rows than the
 * prepared kernels cover (8) run them over consecutive
 * row blocks.  Free with tml_hip_prepared_free.  No counterpart in the
 * reference. */
int tml_hip_prepare_rows_dev(int fmt, int64_t K, int64_t N, const void *W, int64_t ldw, float scale, void *stream,
                             tml_prepared_t *out);
int tml_hip_prepared_free(tml_prepared_t w);
/* tml_hip_gemm_prepared with the fused epilogue of tml_hip_gemm_ex_dev
 * (residual and activation after the bias). */
int tml_hip_gemm_prepared_ex(tml_prepared_t w, int64_t M, const float *A, const float *bias, const float *residual,
                             int act, float *C, float alpha, float beta, void *stream);

/* ----------------------------------------------------------- .tl files */

/* A parsed .tl file: ModelLoader (src/core/loader.zig:41-622).  Parsing and
 * validation run on the host with the reference's checks and error codes;
 * payloads go to HBM byte for byte, so a resident tensor equals the one the
 * reference builds in host memory.
 *
 * tml_tl_open        ModelLoader.init (:55-91): reads the whole file.
 * tml_tl_open_bytes  ModelLoader.initFromBytes (:94-111): borrows `data`,
 *                    which must outlive the handle.
 * tml_tl_close       deinit (:114-131).
 * tml_tl_format      getQuantFormat (:582-585): TML_FMT_* (= the header's
 *                    quant-format byte), or a negative error.
 * tml_tl_count       tensorCount (:587-590): distinct names.
 * tml_tl_name        listTensors()[i] (:592-595), file order; NULL past the
 *                    end.  The string lives as long as the handle.
 * tml_tl_info        getTensorInfo (:597-600): rank (ndim), up to `cap`
 *                    dims, payload offset and size in bytes. */
typedef struct tml_tl_file *tml_tl_t;
int tml_tl_open(const char *path, tml_tl_t *out);
int tml_tl_open_bytes(const void *data, uint64_t size, tml_tl_t *out);
int tml_tl_close(tml_tl_t f);
int tml_tl_format(tml_tl_t f);
int64_t tml_tl_count(tml_tl_t f);
const char *tml_tl_name(tml_tl_t f, int64_t i);
int tml_tl_info(tml_tl_t f, const char *name, int64_t *dims, int cap, int *ndim, uint64_t *offset,
                uint64_t *size);

/* The typed getters, with the reference's checks in its order:
 *   getter TML_FMT_F32   getTensor (:225-264)            data: n f32
 *          TML_FMT_Q8_0  getQuantizedTensorQ8 (:267-307)  data: n int8,   *scale
 *          TML_FMT_Q4_0  getQuantizedTensorQ4 (:310-350)  data: ceil(n/2) packed bytes, *scale
 *          TML_FMT_Q8_K  getQuantizedTensorQ8K (:354-403) data: n int8,   scales: ceil(n/32) f32
 *          TML_FMT_F16   getF16Tensor (:406-437)          data: n binary16
 * n = product of the tensor's dims.  The quantized getters and getF16Tensor
 * fail with TML_ERR_UNSUPPORTED_QUANT_FORMAT on a file of another format;
 * an unknown name is TML_ERR_TENSOR_NOT_FOUND; a payload outside the file
 * or of the wrong size (or a Q8_K block count that does not match) is
 * TML_ERR_CORRUPTED_FILE.  Unused outputs may be NULL.
 * tml_tl_read       host destinations (no GPU needed).
 * tml_tl_read_dev   device destinations, asynchronous on `stream`; the
 *                   handle must stay open until the stream has run them. */
int tml_tl_read(tml_tl_t f, const char *name, int getter, void *data, float *scales, float *scale);
int tml_tl_read_dev(tml_tl_t f, const char *name, int getter, void *data, float *scales, float *scale,
                    void *stream);

/* getTensorDequantized (:442-569) on the device: out receives n f32 values,
 * f32(q) * scale per element (Q8_0 / Q4_0 / Q8_K with its per-32 scales),
 * the exact widening for F16, the values themselves for F32.  Asynchronous;
 * the handle must stay open until the stream has run it. */
int tml_tl_read_dequantized_dev(tml_tl_t f, const char *name, float *out, void *stream);

/* The XLM-R loaders loadQuantizedTransposedQ8 / Q4 / Q8K
 * (src/models/xlm_roberta_punctuation/model.zig:1272-1362) on the device:
 * dequantize q [rows, cols] (the PyTorch [out, in] layout), transpose to
 * [cols, rows] (= [in, out], the matmul's [K, N]) and quantize again with
 * the reference quantizer of the same format, bit for bit.  fmt Q8_0 / Q4_0
 * (per-tensor `scale` in, scales_out[0] out) or Q8_K (`scales` in,
 * ceil(rows*cols/32) scales out).  Device pointers, asynchronous. */
int tml_hip_transpose_requant_dev(int fmt, int64_t rows, int64_t cols, const void *q, const float *scales,
                                  float scale, void *q_out, float *scales_out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TOMOUL_HIP_H */
