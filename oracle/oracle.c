/*
 * oracle.c -- CPU restatement of Tomoul's matrix-multiply hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (tomoul_amd/, include/)
 * links, loads or calls this file.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it, and only as the checker / the timed CPU
 * baseline, never as the thing measured or shipped.
 *
 * Every function names the reference lines it restates (paths relative to the
 * tomoul/tomoul checkout).  The reference is Zig; its default float mode is
 * strict IEEE (no FMA contraction), so this file is compiled with
 * -ffp-contract=off and every multiply and add is rounded separately, in the
 * same order as the reference loops.
 *
 * Pinning (how each function is checked, see tests/test_oracle.py):
 *   orc_matmul_f32 / _naive / _mt   reference KATs (ops.zig:937-1046,
 *                                   main.zig:141-148), exact small-integer
 *                                   products, f64 brute force, blocked ==
 *                                   naive bitwise.
 *   orc_matmul_bias_f32             addBiasInPlace KAT (ops.zig:2629-2654),
 *                                   == matmul + separate bias bitwise.
 *   orc_sgemm                       alpha/beta closed forms (cblas contract,
 *                                   blas.zig:68-94).
 *   orc_matvec                      matvec KAT [14,32] (ops.zig:1048-1076).
 *   orc_quantize_* / orc_dequantize_* / orc_q4_get / orc_q4_set
 *                                   quantizer KATs (quantization.zig:963-1038,
 *                                   1120-1144, 1150-1255, 1337-1453), the
 *                                   half-away-from-zero tie rule, |q| bounds,
 *                                   round-trip <= scale/2.
 *   orc_matmul_q8 / _q8k / _q4      accuracy KATs (quantization.zig:1040-1083,
 *                                   1257-1300, 1455-1492, 1570-1719) and
 *                                   bitwise equality with orc_matmul_f32 on the
 *                                   dequantized weights (the reference's own
 *                                   definition of the scalar path).
 *   orc_f32_to_f16 / orc_f16_to_f32 numpy's IEEE binary16 conversions
 *                                   bitwise: all 65536 halves exhaustively,
 *                                   and f32 -> f16 (round to nearest even)
 *                                   on ties, subnormals, overflow and a large
 *                                   random sample.
 *   orc_matmul_f16                  == orc_matmul_f32 on the widened weight,
 *                                   bitwise (the reference's own definition of
 *                                   its scalar path).
 *   orc_erf_as                      |erf_as - erf| <= the published A&S
 *                                   7.1.26 bound (1.5e-7) plus rounding over a
 *                                   dense grid, odd symmetry, erf(0) = 0.
 *   orc_gelu_exact                  == x/2 (1 + erf(x/sqrt 2)) within the erf
 *                                   bound, GELU(0) = 0, GELU(x) - GELU(-x) = x.
 *   orc_gelu_tanh                   reference KAT (ops.zig:2456-2480, 5
 *                                   elements = all scalar tail), tail ==
 *                                   exact tanh-GELU, vector part: odd,
 *                                   derivative 1 at 0, saturates exactly at
 *                                   inner = 3 (the Pade form's (x-3)^3 root).
 *   orc_fill_normal                 SplitMix64 published output for seed 0,
 *                                   moment checks.  (Input generator, not a
 *                                   reference function.)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef int64_t i64;

/* ------------------------------------------------------------------------ */
/* Seeded input generator: SplitMix64 -> 53-bit uniform -> Box-Muller (f64)  */
/* ------------------------------------------------------------------------ */

uint64_t orc_splitmix64_next(uint64_t *state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* out[i] = float(mean + std * N(0,1)); normals come in Box-Muller pairs
 * (cos, sin) from two consecutive uniforms u1, u2 with u1 mapped to (0,1]. */
void orc_fill_normal(uint64_t seed, i64 n, double mean, double std, float *out) {
    uint64_t st = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (i64 i = 0; i < n; i += 2) {
        double u1 = 1.0 - (double)(orc_splitmix64_next(&st) >> 11) * 0x1.0p-53;
        double u2 = (double)(orc_splitmix64_next(&st) >> 11) * 0x1.0p-53;
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(mean + std * (r * cos(two_pi * u2)));
        if (i + 1 < n) out[i + 1] = (float)(mean + std * (r * sin(two_pi * u2)));
    }
}

/* ------------------------------------------------------------------------ */
/* fp32 GEMM: C[M,N] = A[M,K] . B[K,N], all row-major                        */
/* ------------------------------------------------------------------------ */

/* Plain restatement of one output element of the reference fallback:
 * acc = 0; for k ascending: acc += a[i,k] * b[k,j]   (ops.zig:291-393,
 * 398-412, 556-577).  All fallback branches (4x24 micro-kernel, 4x8, scalar
 * tails, matmulRowRange) perform exactly this per-element sequence. */
void orc_matmul_f32_naive(i64 M, i64 N, i64 K, const float *A, const float *B, float *C) {
    for (i64 i = 0; i < M; i++)
        for (i64 j = 0; j < N; j++) {
            float acc = 0.0f;
            for (i64 k = 0; k < K; k++) acc += A[i * K + k] * B[k * N + j];
            C[i * N + j] = acc;
        }
}

typedef float v8f __attribute__((vector_size(32)));

static inline v8f ld8(const float *p) { v8f v; memcpy(&v, p, sizeof v); return v; }
static inline void st8(float *p, v8f v) { memcpy(p, &v, sizeof v); }
static inline v8f splat8(float x) { v8f v = {x, x, x, x, x, x, x, x}; return v; }

/* Rows [r0, r1) of the register-blocked fallback (ops.zig:277-414):
 * MR = 4 rows, NR = 3 * VEC = 24 columns with VEC = 8 (x86-64, ops.zig:6-11),
 * B streamed one k-row at a time, then a 4x8 block, then scalar columns, then
 * single leftover rows.  Identical arithmetic to orc_matmul_f32_naive. */
static void fallback_rows(i64 r0, i64 r1, i64 n, i64 k, const float *A, const float *B, float *C) {
    const i64 MR = 4, VEC = 8, NR = 24;
    i64 i = r0;
    for (; i + MR <= r1; i += MR) {
        i64 j = 0;
        for (; j + NR <= n; j += NR) {
            v8f c00 = splat8(0), c01 = splat8(0), c02 = splat8(0);
            v8f c10 = splat8(0), c11 = splat8(0), c12 = splat8(0);
            v8f c20 = splat8(0), c21 = splat8(0), c22 = splat8(0);
            v8f c30 = splat8(0), c31 = splat8(0), c32 = splat8(0);
            for (i64 kk = 0; kk < k; kk++) {
                v8f a0 = splat8(A[(i + 0) * k + kk]), a1 = splat8(A[(i + 1) * k + kk]);
                v8f a2 = splat8(A[(i + 2) * k + kk]), a3 = splat8(A[(i + 3) * k + kk]);
                const float *bp = B + kk * n + j;
                v8f b0 = ld8(bp), b1 = ld8(bp + VEC), b2 = ld8(bp + 2 * VEC);
                c00 += a0 * b0; c01 += a0 * b1; c02 += a0 * b2;
                c10 += a1 * b0; c11 += a1 * b1; c12 += a1 * b2;
                c20 += a2 * b0; c21 += a2 * b1; c22 += a2 * b2;
                c30 += a3 * b0; c31 += a3 * b1; c32 += a3 * b2;
            }
            float *cp = C + i * n + j;
            st8(cp, c00); st8(cp + VEC, c01); st8(cp + 2 * VEC, c02); cp += n;
            st8(cp, c10); st8(cp + VEC, c11); st8(cp + 2 * VEC, c12); cp += n;
            st8(cp, c20); st8(cp + VEC, c21); st8(cp + 2 * VEC, c22); cp += n;
            st8(cp, c30); st8(cp + VEC, c31); st8(cp + 2 * VEC, c32);
        }
        for (; j + VEC <= n; j += VEC) {
            v8f c0 = splat8(0), c1 = splat8(0), c2 = splat8(0), c3 = splat8(0);
            for (i64 kk = 0; kk < k; kk++) {
                v8f bv = ld8(B + kk * n + j);
                c0 += splat8(A[(i + 0) * k + kk]) * bv;
                c1 += splat8(A[(i + 1) * k + kk]) * bv;
                c2 += splat8(A[(i + 2) * k + kk]) * bv;
                c3 += splat8(A[(i + 3) * k + kk]) * bv;
            }
            st8(C + (i + 0) * n + j, c0); st8(C + (i + 1) * n + j, c1);
            st8(C + (i + 2) * n + j, c2); st8(C + (i + 3) * n + j, c3);
        }
        for (; j < n; j++) {
            float c0 = 0, c1 = 0, c2 = 0, c3 = 0;
            for (i64 kk = 0; kk < k; kk++) {
                float bv = B[kk * n + j];
                c0 += A[(i + 0) * k + kk] * bv; c1 += A[(i + 1) * k + kk] * bv;
                c2 += A[(i + 2) * k + kk] * bv; c3 += A[(i + 3) * k + kk] * bv;
            }
            C[(i + 0) * n + j] = c0; C[(i + 1) * n + j] = c1;
            C[(i + 2) * n + j] = c2; C[(i + 3) * n + j] = c3;
        }
    }
    for (; i < r1; i++) {
        i64 j = 0;
        for (; j + VEC <= n; j += VEC) {
            v8f c = splat8(0);
            for (i64 kk = 0; kk < k; kk++) c += splat8(A[i * k + kk]) * ld8(B + kk * n + j);
            st8(C + i * n + j, c);
        }
        for (; j < n; j++) {
            float c = 0;
            for (i64 kk = 0; kk < k; kk++) c += A[i * k + kk] * B[kk * n + j];
            C[i * n + j] = c;
        }
    }
}

/* ops.matmul fallback, single-threaded as in the reference (ops.zig:277-414;
 * matmulParallel's fallback is single-threaded too, ops.zig:520-522). */
void orc_matmul_f32(i64 M, i64 N, i64 K, const float *A, const float *B, float *C) {
    fallback_rows(0, M, N, K, A, B, C);
}

/* The same kernel with rows split over `nthreads` OpenMP threads in blocks of
 * 4 (the reference caps its pool at 4 threads, context.zig:285).  Per-element
 * arithmetic is unchanged, so the result is bitwise equal to orc_matmul_f32. */
void orc_matmul_f32_mt(i64 M, i64 N, i64 K, const float *A, const float *B, float *C, int nthreads) {
    i64 nblk = (M + 3) / 4;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (i64 b = 0; b < nblk; b++) {
        i64 r0 = b * 4, r1 = r0 + 4 < M ? r0 + 4 : M;
        fallback_rows(r0, r1, N, K, A, B, C);
    }
}

/* ops.matmulBias fallback (ops.zig:446-468): GEMM into C, then C[i,j] +=
 * bias[j] as a separate rounded add. */
void orc_matmul_bias_f32(i64 M, i64 N, i64 K, const float *A, const float *B, const float *bias, float *C) {
    fallback_rows(0, M, N, K, A, B, C);
    for (i64 i = 0; i < M; i++)
        for (i64 j = 0; j < N; j++) C[i * N + j] += bias[j];
}

/* cblas_sgemm(RowMajor, NoTrans, NoTrans, M, N, K, alpha, A, K, B, N, beta,
 * C, N) semantics as bound by blas.zig:68-94: C = alpha*(A.B) + beta*C, with
 * C's input ignored when beta == 0 (BLAS convention). */
void orc_sgemm(i64 M, i64 N, i64 K, const float *A, const float *B, float *C, float alpha, float beta) {
    float *T = (float *)malloc(sizeof(float) * (size_t)(M * N > 0 ? M * N : 1));
    fallback_rows(0, M, N, K, A, B, T);
    for (i64 i = 0; i < M * N; i++) {
        float ab = alpha * T[i];
        C[i] = beta == 0.0f ? ab : ab + beta * C[i];
    }
    free(T);
}

/* Same product accumulated in f64 (for error reporting, not a reference path). */
void orc_matmul_f64(i64 M, i64 N, i64 K, const float *A, const float *B, double *C) {
    for (i64 i = 0; i < M; i++) {
        double *cr = C + i * N;
        for (i64 j = 0; j < N; j++) cr[j] = 0.0;
        for (i64 k = 0; k < K; k++) {
            double a = A[i * K + k];
            const float *br = B + k * N;
            for (i64 j = 0; j < N; j++) cr[j] += a * (double)br[j];
        }
    }
}

/* ops.matvec non-zblas path (ops.zig:611-642): y[i] = sum_j A[i,j] x[j]. */
void orc_matvec(i64 M, i64 N, const float *A, const float *x, float *y) {
    for (i64 i = 0; i < M; i++) {
        float d = 0.0f;
        for (i64 j = 0; j < N; j++) d += A[i * N + j] * x[j];
        y[i] = d;
    }
}

/* ------------------------------------------------------------------------ */
/* Quantizers (Zig, quantization.zig)                                        */
/* ------------------------------------------------------------------------ */

/* Zig @round on f32 rounds half away from zero, as C roundf does. */
static inline float zround(float x) { return roundf(x); }
static inline float zclamp(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }

static float max_abs_of(const float *v, i64 n) {
    float m = 0.0f;
    for (i64 i = 0; i < n; i++) {
        float a = fabsf(v[i]);
        if (a > m) m = a;
    }
    return m;
}

/* quantizeQ8 (quantization.zig:98-129): per-tensor scale = max|v|/127,
 * q = clamp(round(v * (127/max)), -127, 127); all-zero -> scale 1, q = 0. */
void orc_quantize_q8(i64 n, const float *v, int8_t *q, float *scale) {
    float mx = max_abs_of(v, n);
    if (mx == 0.0f) {
        *scale = 1.0f;
        memset(q, 0, (size_t)n);
        return;
    }
    *scale = mx / 127.0f;
    float inv = 127.0f / mx;
    for (i64 i = 0; i < n; i++) q[i] = (int8_t)zclamp(zround(v[i] * inv), -127.0f, 127.0f);
}

/* dequantizeQ8 (quantization.zig:133-142). */
void orc_dequantize_q8(i64 n, const int8_t *q, float scale, float *out) {
    for (i64 i = 0; i < n; i++) out[i] = (float)q[i] * scale;
}

/* quantizeQ8K (quantization.zig:406-446): one scale per 32 consecutive
 * flattened elements, num_blocks = ceil(n/32); the tail block is short. */
void orc_quantize_q8k(i64 n, const float *v, int8_t *q, float *scales) {
    const i64 BS = 32;
    for (i64 b = 0; b * BS < n; b++) {
        i64 s = b * BS, e = s + BS < n ? s + BS : n;
        float mx = max_abs_of(v + s, e - s);
        if (mx == 0.0f) {
            scales[b] = 1.0f;
            for (i64 i = s; i < e; i++) q[i] = 0;
        } else {
            scales[b] = mx / 127.0f;
            float inv = 127.0f / mx;
            for (i64 i = s; i < e; i++) q[i] = (int8_t)zclamp(zround(v[i] * inv), -127.0f, 127.0f);
        }
    }
}

/* dequantizeQ8K (quantization.zig:449-467). */
void orc_dequantize_q8k(i64 n, const int8_t *q, const float *scales, i64 block, float *out) {
    for (i64 i = 0; i < n; i++) out[i] = (float)q[i] * scales[i / block];
}

/* QuantizedTensorQ4.get (quantization.zig:682-695) with signExtend4
 * (714-717): element 2j is the low nibble of byte j, 2j+1 the high nibble;
 * the nibble is a two's-complement i4, so 0x8 reads back as -8. */
int8_t orc_q4_get(const uint8_t *packed, i64 idx) {
    uint8_t b = packed[idx / 2];
    uint8_t nib = (idx % 2 == 0) ? (uint8_t)(b & 0x0F) : (uint8_t)(b >> 4);
    return (int8_t)((nib & 0x08) ? (int)nib - 16 : (int)nib);
}

/* QuantizedTensorQ4.set (quantization.zig:698-710): clamps to [-7, 7]. */
void orc_q4_set(uint8_t *packed, i64 idx, int8_t value) {
    int v = value < -7 ? -7 : (value > 7 ? 7 : value);
    uint8_t nib = (uint8_t)(v & 0x0F);
    i64 bi = idx / 2;
    if (idx % 2 == 0) packed[bi] = (uint8_t)((packed[bi] & 0xF0) | nib);
    else packed[bi] = (uint8_t)((packed[bi] & 0x0F) | (uint8_t)(nib << 4));
}

/* quantizeQ4 (quantization.zig:721-754): packed bytes zeroed, scale =
 * max|v|/7, q = clamp(round(v * (7/max)), -7, 7); all-zero -> scale 1. */
void orc_quantize_q4(i64 n, const float *v, uint8_t *packed, float *scale) {
    memset(packed, 0, (size_t)((n + 1) / 2));
    float mx = max_abs_of(v, n);
    if (mx == 0.0f) {
        *scale = 1.0f;
        return;
    }
    *scale = mx / 7.0f;
    float inv = 7.0f / mx;
    for (i64 i = 0; i < n; i++) orc_q4_set(packed, i, (int8_t)zclamp(zround(v[i] * inv), -7.0f, 7.0f));
}

/* dequantizeQ4 (quantization.zig:758-768). */
void orc_dequantize_q4(i64 n, const uint8_t *packed, float scale, float *out) {
    for (i64 i = 0; i < n; i++) out[i] = (float)orc_q4_get(packed, i) * scale;
}

/* ------------------------------------------------------------------------ */
/* Weight-only quantized matmuls (scalar oracles)                            */
/* ------------------------------------------------------------------------ */

/* matmulF32Q8 (quantization.zig:158-203): C zeroed, then i, k, j:
 * c[i,j] += a[i,k] * (f32(q[k,j]) * s). */
void orc_matmul_q8(i64 M, i64 N, i64 K, const float *A, const int8_t *q, float s, float *C) {
    memset(C, 0, sizeof(float) * (size_t)(M * N));
    for (i64 i = 0; i < M; i++)
        for (i64 k = 0; k < K; k++) {
            float a = A[i * K + k];
            const int8_t *qr = q + k * N;
            float *cr = C + i * N;
            for (i64 j = 0; j < N; j++) cr[j] += a * ((float)qr[j] * s);
        }
}

/* matmulF32Q8K (quantization.zig:477-525): the scale of weight (k, j) is
 * scales[(k*N + j) / block]. */
void orc_matmul_q8k(i64 M, i64 N, i64 K, const float *A, const int8_t *q, const float *scales, i64 block,
                    float *C) {
    memset(C, 0, sizeof(float) * (size_t)(M * N));
    for (i64 i = 0; i < M; i++)
        for (i64 k = 0; k < K; k++) {
            float a = A[i * K + k];
            float *cr = C + i * N;
            for (i64 j = 0; j < N; j++) {
                i64 w = k * N + j;
                cr[j] += a * ((float)q[w] * scales[w / block]);
            }
        }
}

/* matmulF32Q4 (quantization.zig:778-824): weight (k, j) = get(k*N + j). */
void orc_matmul_q4(i64 M, i64 N, i64 K, const float *A, const uint8_t *packed, float s, float *C) {
    memset(C, 0, sizeof(float) * (size_t)(M * N));
    for (i64 i = 0; i < M; i++)
        for (i64 k = 0; k < K; k++) {
            float a = A[i * K + k];
            float *cr = C + i * N;
            for (i64 j = 0; j < N; j++) cr[j] += a * ((float)orc_q4_get(packed, k * N + j) * s);
        }
}

/* Row-parallel versions of the three loops above for the timed CPU baseline
 * (rows are independent, so results are bitwise unchanged). */
void orc_matmul_q8_mt(i64 M, i64 N, i64 K, const float *A, const int8_t *q, float s, float *C, int nthreads) {
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (i64 i = 0; i < M; i++) orc_matmul_q8(1, N, K, A + i * K, q, s, C + i * N);
}

void orc_matmul_q4_mt(i64 M, i64 N, i64 K, const float *A, const uint8_t *packed, float s, float *C,
                      int nthreads) {
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (i64 i = 0; i < M; i++) orc_matmul_q4(1, N, K, A + i * K, packed, s, C + i * N);
}

/* ------------------------------------------------------------------------ */
/* F16 weights                                                               */
/* ------------------------------------------------------------------------ */

/* toF16 (quantization.zig:1907-1917): Zig's @floatCast f32 -> f16, IEEE
 * round to nearest even; overflow to infinity; NaN stays NaN (quiet). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520: rounds past 65504 */
    if (ax < 0x38800000u) {                                   /* below 2^-14: subnormal or zero */
        int e = (int)(ax >> 23);
        if (e < 102) return (uint16_t)sign;                    /* below 2^-25: rounds to zero */
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        int shift = 126 - e;                                   /* 14..24 */
        uint32_t r = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (ax - 0x38000000u) >> 13, rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

/* @floatCast f16 -> f32: exact. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
    if (e == 0) {
        float v = ldexpf((float)m, -24);
        return sign ? -v : v;
    }
    bits = e == 31 ? (sign | 0x7F800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

void orc_to_f16(i64 n, const float *v, uint16_t *h) {
    for (i64 i = 0; i < n; i++) h[i] = orc_f32_to_f16(v[i]);
}

void orc_from_f16(i64 n, const uint16_t *h, float *v) {
    for (i64 i = 0; i < n; i++) v[i] = orc_f16_to_f32(h[i]);
}

/* matmulF32F16 fallback (quantization.zig:1949-1958): C zeroed, then i, k,
 * j: c[i,j] += a[i,k] * f32(b[k,j]). */
void orc_matmul_f16(i64 M, i64 N, i64 K, const float *A, const uint16_t *B, float *C) {
    memset(C, 0, sizeof(float) * (size_t)(M * N));
    for (i64 i = 0; i < M; i++)
        for (i64 k = 0; k < K; k++) {
            float a = A[i * K + k];
            const uint16_t *br = B + k * N;
            float *cr = C + i * N;
            for (i64 j = 0; j < N; j++) cr[j] += a * orc_f16_to_f32(br[j]);
        }
}

/* ------------------------------------------------------------------------ */
/* Activations of the fused epilogue                                         */
/* ------------------------------------------------------------------------ */

/* erf by Abramowitz & Stegun 7.1.26 (ops.zig:2000-2022). */
float orc_erf_as(float x) {
    const float a1 = 0.254829592f, a2 = -0.284496736f, a3 = 1.421413741f;
    const float a4 = -1.453152027f, a5 = 1.061405429f, p = 0.3275911f;
    float sign = x < 0.0f ? -1.0f : 1.0f;
    float ax = fabsf(x);
    float t = 1.0f / (1.0f + p * ax);
    float t2 = t * t, t3 = t2 * t, t4 = t3 * t, t5 = t4 * t;
    float poly = a1 * t + a2 * t2 + a3 * t3 + a4 * t4 + a5 * t5;
    return sign * (1.0f - poly * expf(-ax * ax));
}

/* geluExact (ops.zig:2029-2057), in place: x * 0.5 * (1 + erf(x / sqrt 2)).
 * The 8-wide and scalar loops compute the same expression. */
void orc_gelu_exact(i64 n, float *v) {
    const float inv_sqrt_2 = 0.7071067811865476f;
    for (i64 i = 0; i < n; i++) {
        float x = v[i];
        v[i] = x * 0.5f * (1.0f + orc_erf_as(x * inv_sqrt_2));
    }
}

/* gelu, tanh form (ops.zig:1947-1998), in place.  Elements below
 * n - n % 8 (the 8-wide AVX2 loop) use the clamped rational form
 * x(27 + x^2) / (27 + 9x^2) for tanh; the scalar tail uses tanh itself. */
void orc_gelu_tanh(i64 n, float *v) {
    const float s2pi = 0.7978845608f, coeff = 0.044715f;
    i64 tail0 = n - n % 8;
    for (i64 i = 0; i < n; i++) {
        float x = v[i];
        float x3 = x * x * x;
        float inner = s2pi * (x + coeff * x3);
        float th;
        if (i < tail0) {
            float i2 = inner * inner;
            th = inner * (27.0f + i2) / (27.0f + 9.0f * i2);
            th = th > 1.0f ? 1.0f : (th < -1.0f ? -1.0f : th);
        } else {
            th = tanhf(inner);
        }
        v[i] = 0.5f * x * (1.0f + th);
    }
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
