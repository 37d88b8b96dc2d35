/* xt_oracle.c - CPU restatement of the reference's FP8 / EVA02-L path. TEST INFRASTRUCTURE ONLY: the product never
 * links, loads or calls this file; tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it as the
 * checker. Built with -O2 -ffp-contract=off (no fast-math): every fused multiply-add is an explicit fmaf().
 * Conventions and the reference lines each part follows are in xt_oracle.h.
 */
#include "xt_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__x86_64__)
#include <immintrin.h>
#endif

static inline uint32_t f2u(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static inline float u2f(uint32_t u)
{
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ---------------------------------------------------------------------------------------------------------------
 * E4M3 codec. OCP E4M3 "fn": bias 7, 3 mantissa bits, subnormals m/8 * 2^-6, max finite 448 (0x7E), 0x7F NaN.
 * Encode = round to nearest even, then saturate to +-448 (kern_common.cuh:99 __NV_SATFINITE; export_eva.py:65
 * clips to +-448 before the RNE cast, which is the same map for finite inputs).
 * ------------------------------------------------------------------------------------------------------------- */
uint8_t xo_e4m3_encode(float x)
{
    uint32_t u, a, e, m, keep, rem;
    uint8_t sign;
    float ax, q;

    u = f2u(x);
    sign = (uint8_t)((u >> 24) & 0x80);
    a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7f;          /* NaN stays NaN */
    ax = u2f(a);
    if (ax >= 448.0f) return sign | 0x7e;             /* saturate (covers +-inf) */
    if (ax < 0x1p-6f) {                               /* subnormal range: multiples of 2^-9 */
        q = nearbyintf(ax * 512.0f);                  /* exact scaling, RNE to an integer 0..8 */
        return sign | (uint8_t)q;                     /* 8 -> 0x08 = 2^-6, the smallest normal */
    }
    e = (a >> 23) - 127;                              /* unbiased exponent, -6..8 */
    m = a & 0x7fffffu;
    keep = m >> 20;
    rem = m & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (keep & 1))) keep++;
    if (keep == 8) {
        keep = 0;
        e++;
    }
    return sign | (uint8_t)(((e + 7) << 3) | keep);
}

float xo_e4m3_decode(uint8_t b)
{
    int s, e, m;
    float v;

    s = b >> 7;
    e = (b >> 3) & 15;
    m = b & 7;
    if (e == 15 && m == 7) return NAN;
    v = e ? ldexpf(1.0f + m / 8.0f, e - 7) : ldexpf(m / 8.0f, -6);
    return s ? -v : v;
}

void xo_e4m3_encode_bits(uint32_t first, uint32_t count, uint8_t *out, int threads)
{
    int64_t i;

#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for num_threads(threads) schedule(static)
#else
    (void)threads;
#endif
    for (i = 0; i < (int64_t)count; i++) out[i] = xo_e4m3_encode(u2f(first + (uint32_t)i));
}

void xo_e4m3_encode_n(const float *x, size_t n, uint8_t *out)
{
    size_t i;

    for (i = 0; i < n; i++) out[i] = xo_e4m3_encode(x[i]);
}

/* bf16 / fp16, round to nearest even */
uint16_t xo_f32_to_bf16(float x)
{
    uint32_t u;

    u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1);
    return (uint16_t)(u >> 16);
}

float xo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t xo_f32_to_f16(float x)
{
    uint32_t u, a, sign, e, m, keep, rem, shift;
    float ax;

    u = f2u(x);
    sign = (u >> 16) & 0x8000u;
    a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    ax = u2f(a);
    if (ax < 0x1p-14f) {                                    /* fp16 subnormal: multiples of 2^-24 */
        return (uint16_t)(sign | (uint32_t)nearbyintf(ax * 0x1p24f));
    }
    e = (a >> 23) - 127;
    m = a & 0x7fffffu;
    shift = 13;
    keep = m >> shift;
    rem = m & ((1u << shift) - 1);
    if (rem > (1u << (shift - 1)) || (rem == (1u << (shift - 1)) && (keep & 1))) keep++;
    if (keep == 1024) {
        keep = 0;
        e++;
    }
    return (uint16_t)(sign | ((e + 15) << 10) | keep);
}

float xo_f16_to_f32(uint16_t h)
{
    uint32_t s, e, m;
    float v;

    s = h >> 15;
    e = (h >> 10) & 31;
    m = h & 1023;
    if (e == 31) v = m ? NAN : INFINITY;
    else if (e == 0) v = ldexpf((float)m, -24);
    else v = ldexpf(1.0f + m / 1024.0f, (int)e - 15);
    return s ? -v : v;
}

float xo_block_scale(float amax)
{
    /* export_eva.py:64-66's sc = amax / 448 per block (one IEEE division); a block whose |max| is below 2^-116
     * (where 448 / amax would leave the normal range) is a zero block, scale 1 */
    return amax < 0x1p-116f ? 1.0f : amax / 448.0f;
}

/* ---------------------------------------------------------------------------------------------------------------
 * Packing (export_eva.py:64-66 per tensor -> per block; eva.h:408 + kern_common.cuh:106 for activations)
 * ------------------------------------------------------------------------------------------------------------- */
void xo_quant_act(const float *x, int M, int K, int ldx, uint8_t *q, int ldq, float *s, int lds)
{
    int m, kb, j;
    float amax, sc, inv;
    const float *xr;

    for (m = 0; m < M; m++)
        for (kb = 0; kb < K / 128; kb++) {
            xr = x + (size_t)m * ldx + kb * 128;
            for (j = 0, amax = 0.0f; j < 128; j++) amax = fmaxf(amax, fabsf(xr[j]));
            sc = xo_block_scale(amax);
            inv = 1.0f / sc;
            s[(size_t)kb * lds + m] = sc;
            for (j = 0; j < 128; j++) q[(size_t)m * ldq + kb * 128 + j] = xo_e4m3_encode(xr[j] * inv);
        }
}

void xo_quant_w(const float *w, int N, int K, uint8_t *q, float *s)
{
    int nb, kb, n, k, NB, KB;
    float amax, sc;

    NB = (N + 127) / 128;
    KB = K / 128;
    memset(q, 0, (size_t)NB * 128 * K);
    for (nb = 0; nb < NB; nb++)
        for (kb = 0; kb < KB; kb++) {
            amax = 0.0f;
            for (n = nb * 128; n < nb * 128 + 128 && n < N; n++)
                for (k = kb * 128; k < kb * 128 + 128; k++) amax = fmaxf(amax, fabsf(w[(size_t)n * K + k]));
            sc = xo_block_scale(amax);
            s[(size_t)nb * KB + kb] = sc;
            for (n = nb * 128; n < nb * 128 + 128 && n < N; n++)
                for (k = kb * 128; k < kb * 128 + 128; k++)
                    q[(size_t)n * K + k] = xo_e4m3_encode(w[(size_t)n * K + k] / sc);
        }
}

/* ---------------------------------------------------------------------------------------------------------------
 * Block-scaled GEMM references. The fp64 form follows kcheck.c:117-126 (fp64 loops over decoded E4M3 operands on
 * sampled rows), with the scale product moved inside the K-block sum.
 * ------------------------------------------------------------------------------------------------------------- */
static float E4LUT[256];
static int e4lut_ready;

static void e4lut_init(void)
{
    int i;

    if (e4lut_ready) return;
    for (i = 0; i < 256; i++) E4LUT[i] = xo_e4m3_decode((uint8_t)i);
    e4lut_ready = 1;
}

void xo_gemm_bs_f64_rows(const uint8_t *qa, int lda, const float *sa, int lds, const uint8_t *qw, const float *sw,
                         int N, int K, const int *rows, int nrows, double *out)
{
    int r, n, kb, k, m, KB;
    double acc, part;

    e4lut_init();
    KB = K / 128;
#pragma omp parallel for private(n, kb, k, m, acc, part) schedule(static)
    for (r = 0; r < nrows; r++) {
        m = rows[r];
        for (n = 0; n < N; n++) {
            acc = 0.0;
            for (kb = 0; kb < KB; kb++) {
                part = 0.0;
                for (k = kb * 128; k < kb * 128 + 128; k++)
                    part += (double)E4LUT[qa[(size_t)m * lda + k]] * (double)E4LUT[qw[(size_t)n * K + k]];
                acc += part * (double)sa[(size_t)kb * lds + m] * (double)sw[(size_t)(n / 128) * KB + kb];
            }
            out[(size_t)r * N + n] = acc;
        }
    }
}

/* The tag head's GEMM (kern_common.cuh:679-727 k_headmv, as the build packs it): weight rows carry 1x128 scales of
 * their own, planes sw [K/128][ldw], like activations: C[m][n] = sum_kb sa[kb][m] sw[kb][n] sum_{k in kb} qa qw, fp64. */
void xo_gemm_rr_f64_rows(const uint8_t *qa, int lda, const float *sa, int lds, const uint8_t *qw, const float *sw,
                         int ldw, int N, int K, const int *rows, int nrows, double *out)
{
    int r;

    e4lut_init();
#pragma omp parallel for schedule(static)
    for (r = 0; r < nrows; r++) {
        const int m = rows[r];
        int n, kb, k;
        for (n = 0; n < N; n++) {
            double acc = 0.0;
            for (kb = 0; kb < K / 128; kb++) {
                double part = 0.0;
                for (k = kb * 128; k < kb * 128 + 128; k++)
                    part += (double)E4LUT[qa[(size_t)m * lda + k]] * (double)E4LUT[qw[(size_t)n * K + k]];
                acc += part * (double)sa[(size_t)kb * lds + m] * (double)sw[(size_t)kb * ldw + n];
            }
            out[(size_t)r * N + n] = acc;
        }
    }
}

int xo_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* Scalar "repo convention" loop: one row, all N columns, decoded operands. */
static void gemm_row_scalar(const float *a, const float *wd, const float *sa_row, const float *sw, int N, int K,
                            float *acc)
{
    int n, kb, k, KB;
    float part, sc;

    KB = K / 128;
    for (n = 0; n < N; n++) {
        acc[n] = 0.0f;
        for (kb = 0; kb < KB; kb++) {
            part = 0.0f;
            for (k = kb * 128; k < kb * 128 + 128; k++) part = fmaf(a[k], wd[(size_t)n * K + k], part);
            sc = sa_row[kb] * sw[(size_t)(n / 128) * KB + kb];
            acc[n] = fmaf(part, sc, acc[n]);
        }
    }
}

#if defined(__x86_64__)
/* AVX2 + FMA: 2 rows x 4 columns register block, 8 lanes along k, horizontal sum per K block. */
__attribute__((target("avx2,fma"))) static inline float hsum8(__m256 v)
{
    __m128 lo, hi;

    lo = _mm256_castps256_ps128(v);
    hi = _mm256_extractf128_ps(v, 1);
    lo = _mm_add_ps(lo, hi);
    lo = _mm_add_ps(lo, _mm_movehl_ps(lo, lo));
    lo = _mm_add_ss(lo, _mm_shuffle_ps(lo, lo, 1));
    return _mm_cvtss_f32(lo);
}

__attribute__((target("avx2,fma"))) static void gemm_rows2_avx2(const float *a0, const float *a1, const float *wd,
                                                               const float *sa0, const float *sa1, const float *sw,
                                                               int N, int K, float *acc0, float *acc1)
{
    int n, kb, k, j, KB;
    __m256 c[2][4], va0, va1, vw;
    float sc;

    KB = K / 128;
    for (n = 0; n < N; n += 4) {
        float r0[4] = {0, 0, 0, 0}, r1[4] = {0, 0, 0, 0};
        int nn = N - n < 4 ? N - n : 4;
        for (kb = 0; kb < KB; kb++) {
            for (j = 0; j < 4; j++) c[0][j] = c[1][j] = _mm256_setzero_ps();
            for (k = kb * 128; k < kb * 128 + 128; k += 8) {
                va0 = _mm256_loadu_ps(a0 + k);
                va1 = _mm256_loadu_ps(a1 + k);
                for (j = 0; j < nn; j++) {
                    vw = _mm256_loadu_ps(wd + (size_t)(n + j) * K + k);
                    c[0][j] = _mm256_fmadd_ps(va0, vw, c[0][j]);
                    c[1][j] = _mm256_fmadd_ps(va1, vw, c[1][j]);
                }
            }
            for (j = 0; j < nn; j++) {
                sc = sa0[kb] * sw[(size_t)((n + j) / 128) * KB + kb];
                r0[j] = fmaf(hsum8(c[0][j]), sc, r0[j]);
                sc = sa1[kb] * sw[(size_t)((n + j) / 128) * KB + kb];
                r1[j] = fmaf(hsum8(c[1][j]), sc, r1[j]);
            }
        }
        for (j = 0; j < nn; j++) {
            acc0[n + j] = r0[j];
            acc1[n + j] = r1[j];
        }
    }
}
#endif

void xo_gemm_bs_f32(const uint8_t *qa, int lda, const float *sa, int lds, const uint8_t *qw, const float *sw, int N,
                    int K, int m0, int m1, float *cf, uint16_t *cb, int ldc, int threads, int avx2)
{
    float *wd;
    int KB, m, n, kb, mi;
    size_t i;

    e4lut_init();
    KB = K / 128;
    wd = (float *)malloc((size_t)N * K * sizeof(float));
    if (!wd) return;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for num_threads(threads) schedule(static)
#else
    (void)threads;
#endif
    for (n = 0; n < N; n++)
        for (i = 0; i < (size_t)K; i++) wd[(size_t)n * K + i] = E4LUT[qw[(size_t)n * K + i]];
#ifdef _OPENMP
#pragma omp parallel num_threads(threads) private(m, n, kb, mi)
#endif
    {
        float *a0 = (float *)malloc((size_t)2 * K * sizeof(float));
        float *acc = (float *)malloc((size_t)2 * N * sizeof(float));
        float sar[2][64];
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (m = m0; m < m1; m += 2) {
            int two = (m + 1 < m1) ? 2 : 1;
            for (mi = 0; mi < two; mi++) {
                for (i = 0; i < (size_t)K; i++) a0[(size_t)mi * K + i] = E4LUT[qa[(size_t)(m + mi) * lda + i]];
                for (kb = 0; kb < KB && kb < 64; kb++) sar[mi][kb] = sa[(size_t)kb * lds + m + mi];
            }
#if defined(__x86_64__)
            if (avx2 && two == 2)
                gemm_rows2_avx2(a0, a0 + K, wd, sar[0], sar[1], sw, N, K, acc, acc + N);
            else
#endif
                for (mi = 0; mi < two; mi++) gemm_row_scalar(a0 + (size_t)mi * K, wd, sar[mi], sw, N, K, acc + (size_t)mi * N);
            for (mi = 0; mi < two; mi++)
                for (n = 0; n < N; n++) {
                    if (cf) cf[(size_t)(m + mi) * ldc + n] = acc[(size_t)mi * N + n];
                    if (cb) cb[(size_t)(m + mi) * ldc + n] = xo_f32_to_bf16(acc[(size_t)mi * N + n]);
                }
        }
        free(a0);
        free(acc);
    }
    free(wd);
}

/* ---------------------------------------------------------------------------------------------------------------
 * LayerNorm over 1024 -> E4M3 with 1x128 scales (kern_common.cuh:147-186 k_ln / ln_row<1>: two-pass mean and
 * variance, eps 1e-6, y = (x - mean) * rstd * gamma + beta), restated in the summation order of the device kernel
 * so the packed bytes are comparable bit for bit: lane l of a 64-lane wave owns elements [8l, 8l+8) and
 * [512+8l, 512+8l+8), sums them in that order, and the 64 lane sums meet in an xor butterfly (32, 16, ..., 1).
 * rstd = 1 / sqrt(var + eps) with IEEE sqrt and division (the reference's rsqrtf under fast-math is not restated).
 * ------------------------------------------------------------------------------------------------------------- */
static float wave_sum64(float *v)
{
    float t[64];
    int off, i;

    for (off = 32; off >= 1; off >>= 1) {
        for (i = 0; i < 64; i++) t[i] = v[i] + v[i ^ off];
        memcpy(v, t, sizeof(t));
    }
    return v[0];
}

static inline int ln_elem(int lane, int j) { return j < 8 ? 8 * lane + j : 512 + 8 * lane + (j - 8); }

void xo_ln_quant(const uint16_t *x, const float *g, const float *b, int M, uint8_t *q, float *s, int lds, float *y)
{
    int m;

#pragma omp parallel for schedule(static)
    for (m = 0; m < M; m++) {
        float v[1024], ls[64], yy[1024], mean, var, rstd, d, amax, sc, inv;
        int l, j, kb, e;

        for (e = 0; e < 1024; e++) v[e] = xo_f16_to_f32(x[(size_t)m * 1024 + e]);
        for (l = 0; l < 64; l++) {
            ls[l] = 0.0f;
            for (j = 0; j < 16; j++) ls[l] += v[ln_elem(l, j)];
        }
        mean = wave_sum64(ls) * (1.0f / 1024.0f);
        for (l = 0; l < 64; l++) {
            ls[l] = 0.0f;
            for (j = 0; j < 16; j++) {
                d = v[ln_elem(l, j)] - mean;
                ls[l] = fmaf(d, d, ls[l]);
            }
        }
        var = wave_sum64(ls) * (1.0f / 1024.0f);
        rstd = 1.0f / sqrtf(var + 1e-6f);
        for (e = 0; e < 1024; e++) yy[e] = fmaf((v[e] - mean) * rstd, g[e], b[e]);
        if (y) memcpy(y + (size_t)m * 1024, yy, sizeof(yy));
        for (kb = 0; kb < 8; kb++) {
            for (e = kb * 128, amax = 0.0f; e < kb * 128 + 128; e++) amax = fmaxf(amax, fabsf(yy[e]));
            sc = xo_block_scale(amax);
            inv = 1.0f / sc;
            s[(size_t)kb * lds + m] = sc;
            for (e = kb * 128; e < kb * 128 + 128; e++) q[(size_t)m * 1024 + e] = xo_e4m3_encode(yy[e] * inv);
        }
    }
}

/* kcheck.c:21-22, 106-107: the reference kernel checker's LCG operand generators */
void xo_lcg_frand(uint32_t *rs, size_t n, float *out)
{
    size_t i;

    for (i = 0; i < n; i++) {
        *rs = *rs * 1664525u + 1013904223u;
        out[i] = (float)(*rs >> 8) / 8388608.0f - 1.0f;
    }
}

void xo_lcg_e4m3(uint32_t *rs, size_t n, uint8_t *out)
{
    size_t i;
    uint8_t b;

    for (i = 0; i < n; i++) {
        do {
            *rs = *rs * 1664525u + 1013904223u;
            b = (uint8_t)(*rs >> 24);
        } while ((b & 0x7F) == 0x7F || ((b >> 3) & 15) > 9);
        out[i] = b;
    }
}

/* =================================================================================================================
 * EVA02-L forward pieces
 * =============================================================================================================== */
static float f16f(uint16_t h) { return xo_f16_to_f32(h); }

void xo_qkv_epi(const float *acc, int nb, const float *cs, uint16_t *q, uint16_t *k, uint16_t *vt)
{
    int m, M = nb * XO_T;

#pragma omp parallel for schedule(static)
    for (m = 0; m < M; m++) {
        int b = m / XO_T, t = m % XO_T, part, h, i, d;
        const float *a = acc + (size_t)m * 3072;
        for (part = 0; part < 2; part++) {
            uint16_t *dst = part ? k : q;
            for (h = 0; h < 16; h++)
                for (i = 0; i < 32; i++) {
                    float f0 = a[part * 1024 + h * 64 + 2 * i], f1 = a[part * 1024 + h * 64 + 2 * i + 1], g0;
                    if (t >= 1) {
                        float c = cs[((size_t)(t - 1) * 32 + i) * 2], sn = cs[((size_t)(t - 1) * 32 + i) * 2 + 1];
                        g0 = f0 * c - f1 * sn;
                        f1 = f1 * c + f0 * sn;
                        f0 = g0;
                    }
                    dst[(((size_t)b * 16 + h) * XO_TP + t) * 64 + 2 * i] = xo_f32_to_bf16(f0);
                    dst[(((size_t)b * 16 + h) * XO_TP + t) * 64 + 2 * i + 1] = xo_f32_to_bf16(f1);
                }
        }
        for (h = 0; h < 16; h++)
            for (d = 0; d < 64; d++)
                vt[(((size_t)b * 16 + h) * 64 + d) * XO_TP + t] = xo_f32_to_bf16(a[2048 + h * 64 + d]);
    }
}

void xo_attention_seq(const uint16_t *q, const uint16_t *k, const uint16_t *vt, int nseq, int T, int TP, int qstep,
                      double *o, int threads)
{
    int bh;

    if (qstep < 1) qstep = 1;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
#else
    (void)threads;
#endif
    for (bh = 0; bh < nseq * 16; bh++) {
        int b = bh / 16, h = bh % 16, t, j, d;
        double *Q = (double *)malloc(sizeof(double) * T * 64);
        double *Kd = (double *)malloc(sizeof(double) * T * 64);
        double *V = (double *)malloc(sizeof(double) * T * 64);
        double *s = (double *)malloc(sizeof(double) * T);
        for (t = 0; t < T; t++)
            for (d = 0; d < 64; d++) {
                Q[t * 64 + d] = xo_bf16_to_f32(q[((size_t)bh * TP + t) * 64 + d]);
                Kd[t * 64 + d] = xo_bf16_to_f32(k[((size_t)bh * TP + t) * 64 + d]);
                V[t * 64 + d] = xo_bf16_to_f32(vt[((size_t)bh * 64 + d) * TP + t]);
            }
        for (t = 0; t < T; t += qstep) {
            double mx = -INFINITY, l = 0.0, acc[64];
            for (j = 0; j < T; j++) {
                double a0 = 0, a1 = 0, a2 = 0, a3 = 0;
                for (d = 0; d < 64; d += 4) {
                    a0 += Q[t * 64 + d] * Kd[j * 64 + d];
                    a1 += Q[t * 64 + d + 1] * Kd[j * 64 + d + 1];
                    a2 += Q[t * 64 + d + 2] * Kd[j * 64 + d + 2];
                    a3 += Q[t * 64 + d + 3] * Kd[j * 64 + d + 3];
                }
                s[j] = (a0 + a1) + (a2 + a3);
                if (s[j] > mx) mx = s[j];
            }
            for (d = 0; d < 64; d++) acc[d] = 0.0;
            for (j = 0; j < T; j++) {
                double p = exp2(s[j] - mx);
                l += p;
                for (d = 0; d < 64; d++) acc[d] += p * V[j * 64 + d];
            }
            for (d = 0; d < 64; d++) o[((size_t)b * T + t) * 1024 + h * 64 + d] = acc[d] / l;
        }
        free(Q);
        free(Kd);
        free(V);
        free(s);
    }
}

void xo_attention(const uint16_t *q, const uint16_t *k, const uint16_t *vt, int nb, double *o, int threads)
{
    xo_attention_seq(q, k, vt, nb, XO_T, XO_TP, 1, o, threads);
}

void xo_fc1_epi(const float *acc, int M, float *h, float *stat)
{
    int m;

#pragma omp parallel for schedule(static)
    for (m = 0; m < M; m++) {
        int u, blk;
        for (u = 0; u < XO_HIDP; u++) {
            int c = u / 16, w = u % 16;
            float g = acc[(size_t)m * 2 * XO_HIDP + 32 * c + w], x = acc[(size_t)m * 2 * XO_HIDP + 32 * c + 16 + w];
            float e = expf(-g), den = 1.0f + e, sg = g / den;
            h[(size_t)m * XO_HIDP + u] = sg * x;
        }
        for (blk = 0; blk < XO_HIDP / 128; blk++) {
            float s = 0.0f, q = 0.0f, v;
            for (u = blk * 128; u < blk * 128 + 128; u++) {
                v = h[(size_t)m * XO_HIDP + u];
                s += v;
                q = fmaf(v, v, q);
            }
            stat[((size_t)blk * M + m) * 2] = s;
            stat[((size_t)blk * M + m) * 2 + 1] = q;
        }
    }
}

void xo_fc2_epi(const float *acc, int M, const float *stat, const float *c, const float *d, uint16_t *x)
{
    int m;

#pragma omp parallel for schedule(static)
    for (m = 0; m < M; m++) {
        float S = 0.0f, Q = 0.0f, mean, var, rstd, nm, y;
        int blk, n;
        for (blk = 0; blk < XO_HIDP / 128; blk++) {
            S += stat[((size_t)blk * M + m) * 2];
            Q += stat[((size_t)blk * M + m) * 2 + 1];
        }
        mean = S / (float)XO_HID;
        var = Q / (float)XO_HID - mean * mean;
        var = fmaxf(var, 0.0f);
        rstd = 1.0f / sqrtf(var + 1e-6f);
        nm = -mean * rstd;
        for (n = 0; n < XO_D; n++) {
            y = fmaf(rstd, acc[(size_t)m * XO_D + n], fmaf(nm, c[n], d[n]));
            x[(size_t)m * XO_D + n] = xo_f32_to_f16(f16f(x[(size_t)m * XO_D + n]) + y);
        }
    }
}

void xo_oproj_epi(const float *acc, int M, uint16_t *x)
{
    size_t i;

    for (i = 0; i < (size_t)M * XO_D; i++) x[i] = xo_f32_to_f16(f16f(x[i]) + acc[i]);
}

/* ---- PixAI (ViTDet-L) block epilogues, px_kernels.cu ---- */
void xo_px_qkv_epi(const float *acc, int M, int L, const float *bias, const float *cs, uint16_t *q, uint16_t *k,
                   uint16_t *vt)
{
    int m;

#pragma omp parallel for schedule(static)
    for (m = 0; m < M; m++) {
        int s = m / L, t = m % L, part, h, i, d;
        const float *a = acc + (size_t)m * 3072;
        for (part = 0; part < 2; part++) {
            uint16_t *dst = part ? k : q;
            for (h = 0; h < 16; h++)
                for (i = 0; i < 32; i++) {
                    const int n = part * 1024 + h * 64 + 2 * i;
                    const float f0 = a[n] + bias[n], f1 = a[n + 1] + bias[n + 1];
                    const float c = cs[((size_t)t * 32 + i) * 2], sn = cs[((size_t)t * 32 + i) * 2 + 1];
                    const float g0 = f0 * c - f1 * sn, g1 = f1 * c + f0 * sn;
                    dst[(((size_t)s * 16 + h) * L + t) * 64 + 2 * i] = xo_f32_to_bf16(g0);
                    dst[(((size_t)s * 16 + h) * L + t) * 64 + 2 * i + 1] = xo_f32_to_bf16(g1);
                }
        }
        for (h = 0; h < 16; h++)
            for (d = 0; d < 64; d++)
                vt[(((size_t)s * 16 + h) * 64 + d) * L + t] = xo_f32_to_bf16(a[2048 + h * 64 + d] + bias[2048 + h * 64 + d]);
    }
}

void xo_px_res_epi(const float *acc, int M, const float *bias, uint16_t *x)
{
    size_t i;

    for (i = 0; i < (size_t)M * XO_D; i++) x[i] = xo_f32_to_f16(f16f(x[i]) + (acc[i] + bias[i % XO_D]));
}

void xo_px_fc1_epi(const float *acc, int M, const float *bias, const float *rs, float *h)
{
    int m;

#pragma omp parallel for schedule(static)
    for (m = 0; m < M; m++) {
        int u;
        for (u = 0; u < XO_PX_HID; u++) {
            const float v = acc[(size_t)m * XO_PX_HID + u] + bias[u];
            const float g = v * (0.5f * (1.0f + erff(v * 0.70710678f)));
            h[(size_t)m * XO_PX_HID + u] = rs ? g * rs[u] : g;
        }
    }
}

void xo_px_pe(const uint16_t *in, const uint16_t *pe, int M, uint16_t *x)
{
    int m;

#pragma omp parallel for schedule(static)
    for (m = 0; m < M; m++) {
        int n, k;
        for (n = 0; n < 1024; n++) {
            double a = 0.0;
            for (k = 0; k < 588; k++) a += (double)xo_f16_to_f32(in[(size_t)m * 592 + k]) * xo_f16_to_f32(pe[(size_t)n * 592 + k]);
            x[(size_t)m * 1024 + n] = xo_f32_to_f16((float)a);
        }
    }
}

void xo_px_pembed(const uint16_t *x, int M, int T, const float *pos, const float *g, const float *b, uint16_t *y)
{
    int m;

#pragma omp parallel for schedule(static)
    for (m = 0; m < M; m++) {
        float v[1024], ls[64], mean, var, rstd, d;
        int l, j, e;

        for (e = 0; e < 1024; e++) v[e] = xo_f16_to_f32(x[(size_t)m * 1024 + e]) + pos[(size_t)(m % T) * 1024 + e];
        for (l = 0; l < 64; l++) {
            ls[l] = 0.0f;
            for (j = 0; j < 16; j++) ls[l] += v[ln_elem(l, j)];
        }
        mean = wave_sum64(ls) * (1.0f / 1024.0f);
        for (l = 0; l < 64; l++) {
            ls[l] = 0.0f;
            for (j = 0; j < 16; j++) {
                d = v[ln_elem(l, j)] - mean;
                ls[l] = fmaf(d, d, ls[l]);
            }
        }
        var = wave_sum64(ls) * (1.0f / 1024.0f);
        rstd = 1.0f / sqrtf(var + 1e-5f);
        for (e = 0; e < 1024; e++) y[(size_t)m * 1024 + e] = xo_f32_to_f16(fmaf((v[e] - mean) * rstd, g[e], b[e]));
    }
}

void xo_px_hln(const uint16_t *x, int M, int T, const float *g, const float *b, const uint16_t *hpos, const float *U,
               uint16_t *y, double *s)
{
    int m;

#pragma omp parallel for schedule(static)
    for (m = 0; m < M; m++) {
        float v[1024], ls[64], mean, var, rstd, d;
        int l, j, e, h;

        for (e = 0; e < 1024; e++) v[e] = xo_f16_to_f32(x[(size_t)m * 1024 + e]);
        for (l = 0; l < 64; l++) {
            ls[l] = 0.0f;
            for (j = 0; j < 16; j++) ls[l] += v[ln_elem(l, j)];
        }
        mean = wave_sum64(ls) * (1.0f / 1024.0f);
        for (l = 0; l < 64; l++) {
            ls[l] = 0.0f;
            for (j = 0; j < 16; j++) {
                d = v[ln_elem(l, j)] - mean;
                ls[l] = fmaf(d, d, ls[l]);
            }
        }
        var = wave_sum64(ls) * (1.0f / 1024.0f);
        rstd = 1.0f / sqrtf(var + 1e-5f);
        for (e = 0; e < 1024; e++)
            y[(size_t)m * 1024 + e] =
                xo_f32_to_f16(fmaf((v[e] - mean) * rstd, g[e], b[e]) + xo_f16_to_f32(hpos[(size_t)(m % T) * 1024 + e]));
        for (h = 0; h < 16; h++) {
            double a = 0.0;
            for (e = 0; e < 1024; e++) a += (double)U[h * 1024 + e] * xo_f16_to_f32(y[(size_t)m * 1024 + e]);
            s[(size_t)m * 16 + h] = a;
        }
    }
}

void xo_px_hsoft(const float *s, int nb, int T, double *P)
{
    int bh;

#pragma omp parallel for schedule(static)
    for (bh = 0; bh < nb * 16; bh++) {
        const int b = bh / 16, h = bh % 16;
        double mx = -1e300, l = 0.0;
        int t;
        for (t = 0; t < T; t++) mx = fmax(mx, s[((size_t)b * T + t) * 16 + h]);
        for (t = 0; t < T; t++) l += exp2(s[((size_t)b * T + t) * 16 + h] - mx);
        for (t = 0; t < T; t++) P[(size_t)bh * T + t] = exp2(s[((size_t)b * T + t) * 16 + h] - mx) / l;
    }
}

void xo_px_hpool_hv(const uint16_t *P, const uint16_t *y, int nb, int T, const uint16_t *wv, double *o)
{
    int bh;

#pragma omp parallel for schedule(static)
    for (bh = 0; bh < nb * 16; bh++) {
        const int b = bh / 16, h = bh % 16;
        double pooled[1024];
        int t, d, n;
        for (d = 0; d < 1024; d++) pooled[d] = 0.0;
        for (t = 0; t < T; t++) {
            const double p = xo_f16_to_f32(P[(size_t)bh * T + t]);
            const uint16_t *yr = y + ((size_t)b * T + t) * 1024;
            for (d = 0; d < 1024; d++) pooled[d] += p * xo_f16_to_f32(yr[d]);
        }
        for (n = 0; n < 64; n++) {
            double a = 0.0;
            for (d = 0; d < 1024; d++) a += (double)xo_f16_to_f32(wv[(size_t)(64 * h + n) * 1024 + d]) * pooled[d];
            o[(size_t)b * 1024 + 64 * h + n] = a;
        }
    }
}

void xo_embed(const uint16_t *in, const uint16_t *pe, const float *pos, int nb, uint16_t *x)
{
    int r;
    float *pef = (float *)malloc(sizeof(float) * 1024 * 592);

    for (r = 0; r < 1024 * 592; r++) pef[r] = f16f(pe[r]);
#pragma omp parallel for schedule(static)
    for (r = 0; r < nb * 1024; r++) {
        int b = r / 1024, p = r % 1024, n, kk;
        float a[592];
        for (kk = 0; kk < 592; kk++) a[kk] = f16f(in[(size_t)r * 592 + kk]);
        for (n = 0; n < XO_D; n++) {
            double dot = 0.0;
            for (kk = 0; kk < 592; kk++) dot += (double)a[kk] * (double)pef[(size_t)n * 592 + kk];
            x[((size_t)b * XO_T + 1 + p) * XO_D + n] = xo_f32_to_f16((float)dot + pos[(size_t)(1 + p) * XO_D + n]);
        }
        if (p == 0)
            for (n = 0; n < XO_D; n++) x[(size_t)b * XO_T * XO_D + n] = xo_f32_to_f16(pos[n]);
    }
    free(pef);
}

/* k_pool's order: per column, 32 groups of 32 tokens (1 + 32 g .. 32 g + 32) each summed in token order, the group
 * sums added in group order, times 1/1024 (eva_kernels.cu:402-431 computes the same mean with its own grouping) */
void xo_pool(const uint16_t *x, int nb, float *p)
{
    int b, n, g, t;

    for (b = 0; b < nb; b++)
        for (n = 0; n < XO_D; n++) {
            float tot = 0.0f;
            for (g = 0; g < 32; g++) {
                float s = 0.0f;
                for (t = 0; t < 32; t++) s += f16f(x[((size_t)b * XO_T + 1 + 32 * g + t) * XO_D + n]);
                tot = g ? tot + s : s;
            }
            p[(size_t)b * XO_D + n] = tot * (1.0f / 1024.0f);
        }
}

/* LayerNorm of one 1024-row in the device order (see xo_ln_quant) */
static void ln_row_dev(const float *v, const float *g, const float *b, float *y)
{
    float ls[64], mean, var, rstd, d;
    int l, j, e;

    for (l = 0; l < 64; l++) {
        ls[l] = 0.0f;
        for (j = 0; j < 16; j++) ls[l] += v[ln_elem(l, j)];
    }
    mean = wave_sum64(ls) * (1.0f / 1024.0f);
    for (l = 0; l < 64; l++) {
        ls[l] = 0.0f;
        for (j = 0; j < 16; j++) {
            d = v[ln_elem(l, j)] - mean;
            ls[l] = fmaf(d, d, ls[l]);
        }
    }
    var = wave_sum64(ls) * (1.0f / 1024.0f);
    rstd = 1.0f / sqrtf(var + 1e-6f);
    for (e = 0; e < 1024; e++) y[e] = fmaf((v[e] - mean) * rstd, g[e], b[e]);
}

void xo_lnh(const float *p, const float *g, const float *b, int nb, uint16_t *pn, uint8_t *q, float *s, int lds)
{
    int r, e;
    float y[1024], yq[1024];

    for (r = 0; r < nb; r++) {
        ln_row_dev(p + (size_t)r * 1024, g, b, y);
        for (e = 0; e < 1024; e++) {
            pn[(size_t)r * 1024 + e] = xo_f32_to_f16(y[e]);
            yq[e] = f16f(pn[(size_t)r * 1024 + e]);
        }
        /* 1x128 packing of the fp16 values; row r of a one-row act quant into the planes */
        {
            int kb;
            for (kb = 0; kb < 8; kb++) {
                float amax = 0.0f, sc, inv;
                for (e = kb * 128; e < kb * 128 + 128; e++) amax = fmaxf(amax, fabsf(yq[e]));
                sc = xo_block_scale(amax);
                inv = 1.0f / sc;
                s[(size_t)kb * lds + r] = sc;
                for (e = kb * 128; e < kb * 128 + 128; e++) q[(size_t)r * 1024 + e] = xo_e4m3_encode(yq[e] * inv);
            }
        }
    }
}

void xo_fold_w2(const uint16_t *w2, int ldw2, const float *gamma, const float *beta, float *wt, float *d)
{
    int n, k;

    for (n = 0; n < XO_D; n++) {
        float dd = 0.0f;
        for (k = 0; k < XO_HIDP; k++) {
            float w = k < XO_HID ? f16f(w2[(size_t)n * ldw2 + k]) : 0.0f;
            wt[(size_t)n * XO_HIDP + k] = k < XO_HID ? w * gamma[k] : 0.0f;
            if (k < XO_HID) dd = fmaf(w, beta[k], dd);
        }
        d[n] = dd;
    }
}

void xo_fold_c(const uint8_t *q, const float *s, float *c)
{
    int n, k;

    e4lut_init();
    for (n = 0; n < XO_D; n++) {
        float cc = 0.0f;
        for (k = 0; k < XO_HIDP; k++)
            cc = fmaf(E4LUT[q[(size_t)n * XO_HIDP + k]], s[(size_t)(n / 128) * (XO_HIDP / 128) + k / 128], cc);
        c[n] = cc;
    }
}

void xo_prune24(uint8_t *q, int N, int K, int wanda)
{
    float *colmax = NULL;
    int n, k;

    e4lut_init();
    if (wanda) {
        colmax = (float *)calloc((size_t)K, sizeof(float));
        for (n = 0; n < N; n++)
            for (k = 0; k < K; k++) {
                const float v = fabsf(E4LUT[q[(size_t)n * K + k]]);
                if (v > colmax[k]) colmax[k] = v;
            }
    }
    for (n = 0; n < N; n++)
        for (k = 0; k < K; k += 4) {
            uint8_t *g = q + (size_t)n * K + k;
            float sc[4];
            int i, j, drop[4] = {0, 0, 0, 0}, nd = 0;
            for (i = 0; i < 4; i++) sc[i] = fabsf(E4LUT[g[i]]) * (wanda ? colmax[k + i] : 1.0f);
            /* the 2 lowest scores in ascending (score, k) order: a stable ascending sort's first two */
            while (nd < 2) {
                int best = -1;
                for (j = 0; j < 4; j++)
                    if (!drop[j] && (best < 0 || sc[j] < sc[best])) best = j;
                drop[best] = 1;
                nd++;
            }
            for (i = 0; i < 4; i++)
                if (drop[i]) g[i] = 0;
        }
    free(colmax);
}

int xo_pack24(const uint8_t *q, int N, int K, uint8_t *vals, uint32_t *idx)
{
    const int KB = K / 128;
    int t, kb, l, j;

    e4lut_init();
    for (t = 0; t < N / 16; t++)
        for (kb = 0; kb < KB; kb++)
            for (l = 0; l < 64; l++) {
                const int g = l >> 4, r = l & 15;
                const uint8_t *row = q + (size_t)(16 * t + r) * K + 128 * kb + 32 * g;
                uint8_t *v = vals + (((size_t)t * KB + kb) * 64 + l) * 16;
                uint32_t w = 0;
                for (j = 0; j < 8; j++) {
                    const uint8_t *grp = row + 4 * j;
                    int pos[2], np = 0, i;
                    for (i = 0; i < 4 && np < 3; i++)
                        if (grp[i] != 0) {
                            if (np == 2) return -1;
                            pos[np++] = i;
                        }
                    for (i = 0; i < 4 && np < 2; i++)  /* complete with the lowest-k zero positions */
                        if (grp[i] == 0 && !(np == 1 && pos[0] == i)) pos[np++] = i;
                    if (pos[0] > pos[1]) { i = pos[0]; pos[0] = pos[1]; pos[1] = i; }
                    v[2 * j] = grp[pos[0]];
                    v[2 * j + 1] = grp[pos[1]];
                    w |= (uint32_t)(pos[0] | pos[1] << 2) << (4 * j);
                }
                idx[((size_t)t * KB + kb) * 64 + l] = w;
            }
    return 0;
}

/* fp16 [rows][ld] (first cols columns) -> fp32 [rows_out][cols_out], zero padded */
static float *f16_to_f32_pad(const uint16_t *w, int rows, int cols, int ld, int rows_out, int cols_out)
{
    float *o = (float *)calloc((size_t)rows_out * cols_out, sizeof(float));
    int r, c;

    for (r = 0; r < rows; r++)
        for (c = 0; c < cols; c++) o[(size_t)r * cols_out + c] = f16f(w[(size_t)r * ld + c]);
    return o;
}

int xo_forward(const xo_model *md, const uint16_t *in, int nb, int nl, float *out, uint16_t *pn, int threads)
{
    const int avx = getenv("XO_SCALAR") ? 0 : 1;
    const int M = nb * XO_T, nt = md->nt;
    uint16_t *x = (uint16_t *)malloc(sizeof(uint16_t) * M * XO_D);
    uint8_t *h8 = (uint8_t *)malloc((size_t)M * XO_HIDP);
    float *hs = (float *)malloc(sizeof(float) * 22 * M);
    float *acc = (float *)malloc(sizeof(float) * (size_t)M * 2 * XO_HIDP);
    float *hf = (float *)malloc(sizeof(float) * (size_t)M * XO_HIDP);
    float *stat = (float *)malloc(sizeof(float) * 22 * M * 2);
    uint16_t *q = (uint16_t *)calloc((size_t)nb * 16 * XO_TP * 64, 2);
    uint16_t *k = (uint16_t *)calloc((size_t)nb * 16 * XO_TP * 64, 2);
    uint16_t *vt = (uint16_t *)calloc((size_t)nb * 16 * XO_TP * 64, 2);
    double *o = (double *)malloc(sizeof(double) * (size_t)M * XO_D);
    float *of = (float *)malloc(sizeof(float) * (size_t)M * XO_D);
    uint8_t *wq = (uint8_t *)malloc((size_t)2 * XO_HIDP * XO_D);
    float *ws = (float *)malloc(sizeof(float) * 44 * 22);
    float *cfold = (float *)malloc(sizeof(float) * XO_D), *dfold = (float *)malloc(sizeof(float) * XO_D);
    float *pool = (float *)malloc(sizeof(float) * nb * XO_D);
    uint8_t *pq = (uint8_t *)malloc((size_t)nb * XO_D);
    float *ps = (float *)malloc(sizeof(float) * 8 * nb);
    double *logit = (double *)malloc(sizeof(double) * nb * nt);
    float *wf;
    int i, r, n;

    xo_embed(in, md->pe, md->pos, nb, x);
    for (i = 0; i < nl; i++) {
        /* attention */
        xo_ln_quant(x, md->ln1w[i], md->ln1b[i], M, h8, hs, M, NULL);
        wf = f16_to_f32_pad(md->wqkv[i], 3072, XO_D, XO_D, 3072, XO_D);
        xo_quant_w(wf, 3072, XO_D, wq, ws);
        free(wf);
        if (md->sparse) xo_prune24(wq, 3072, XO_D, 0);
        xo_gemm_bs_f32(h8, XO_D, hs, M, wq, ws, 3072, XO_D, 0, M, acc, NULL, 3072, threads, avx);
        xo_qkv_epi(acc, nb, md->cs, q, k, vt);
        xo_attention(q, k, vt, nb, o, threads);
        for (r = 0; r < M * XO_D; r++) of[r] = (float)o[r];
        xo_quant_act(of, M, XO_D, XO_D, h8, XO_D, hs, M);
        wf = f16_to_f32_pad(md->wo[i], XO_D, XO_D, XO_D, XO_D, XO_D);
        xo_quant_w(wf, XO_D, XO_D, wq, ws);
        free(wf);
        if (md->sparse) xo_prune24(wq, XO_D, XO_D, 0);
        xo_gemm_bs_f32(h8, XO_D, hs, M, wq, ws, XO_D, XO_D, 0, M, acc, NULL, XO_D, threads, avx);
        xo_oproj_epi(acc, M, x);
        /* MLP */
        xo_ln_quant(x, md->ln2w[i], md->ln2b[i], M, h8, hs, M, NULL);
        wf = f16_to_f32_pad(md->w12[i], 2 * 2736, XO_D, XO_D, 2 * XO_HIDP, XO_D);
        xo_quant_w(wf, 2 * XO_HIDP, XO_D, wq, ws);
        free(wf);
        if (md->sparse) xo_prune24(wq, 2 * XO_HIDP, XO_D, 0);
        xo_gemm_bs_f32(h8, XO_D, hs, M, wq, ws, 2 * XO_HIDP, XO_D, 0, M, acc, NULL, 2 * XO_HIDP, threads, avx);
        xo_fc1_epi(acc, M, hf, stat);
        xo_quant_act(hf, M, XO_HIDP, XO_HIDP, h8, XO_HIDP, hs, M);
        wf = (float *)malloc(sizeof(float) * XO_D * XO_HIDP);
        xo_fold_w2(md->w2[i], 2736, md->mlnw[i], md->mlnb[i], wf, dfold);
        xo_quant_w(wf, XO_D, XO_HIDP, wq, ws);
        free(wf);
        if (md->sparse) xo_prune24(wq, XO_D, XO_HIDP, 0);
        xo_fold_c(wq, ws, cfold);
        xo_gemm_bs_f32(h8, XO_HIDP, hs, M, wq, ws, XO_D, XO_HIDP, 0, M, acc, NULL, XO_D, threads, avx);
        xo_fc2_epi(acc, M, stat, cfold, dfold, x);
    }
    xo_pool(x, nb, pool);
    xo_lnh(pool, md->fnw, md->fnb, nb, pn, pq, ps, nb);
    {   /* the head: every fp16 row packed with its own 1x128 scales, fp64 logits, fp32 sigmoid */
        uint8_t *hq = (uint8_t *)malloc((size_t)nt * XO_D);
        float *hsc = (float *)malloc(sizeof(float) * 8 * nt);
        int *rows = (int *)malloc(sizeof(int) * nb);
        wf = f16_to_f32_pad(md->hw, nt, XO_D, XO_D, nt, XO_D);
        xo_quant_act(wf, nt, XO_D, XO_D, hq, XO_D, hsc, nt);
        free(wf);
        for (r = 0; r < nb; r++) rows[r] = r;
        xo_gemm_rr_f64_rows(pq, XO_D, ps, nb, hq, hsc, nt, nt, XO_D, rows, nb, logit);
        for (r = 0; r < nb; r++)
            for (n = 0; n < nt; n++)
                out[(size_t)r * nt + n] = 1.0f / (1.0f + expf(-((float)logit[(size_t)r * nt + n] + md->hb[n])));
        free(hq);
        free(hsc);
        free(rows);
    }
    free(x); free(h8); free(hs); free(acc); free(hf); free(stat); free(q); free(k); free(vt); free(o); free(of);
    free(wq); free(ws); free(cfold); free(dfold); free(pool); free(pq); free(ps); free(logit);
    return 0;
}
