/* xt_cpugemm.c - the CPU baseline of the block-scaled FP8 GEMM (TEST AND BENCHMARK INFRASTRUCTURE ONLY: loaded by
 * bench.py's cpu_baseline leg and the tests, never by the product).
 *
 * Semantics, the reference's per-tensor alpha * acc (src/engine/eva.h:415-418) generalised to 1x128 activation and
 * 128x128 weight blocks, E4M3 decoded as src/tools/kcheck.c:25-33:
 *   C[m][n] = bf16_rne( sum_kb fma(dot128(A[m][kb], W[n][kb]), sa[kb][m] * sw[n / 128][kb], . ) )
 * The dot of one K block is taken in 8 interleaved fp32 partial sums (k mod 8) added in a fixed tree; every product
 * of two E4M3 values is exact in fp32, so a multiply and an add round once, as an fma would. The promotion is one
 * fmaf per K block.
 *
 * The same source is built twice (Makefile): libcpugemm_scalar.so with -O3 -ffp-contract=off, and libcpugemm_avx2.so
 * with -O3 -mavx2 -mfma -ffp-contract=off, where the 8 partial sums become one ymm register. Work is split over
 * 128-row blocks of M with OpenMP.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* one partial-sum update: the product of two E4M3 values is exact in fp32, so fmaf and a multiply then an add give the
 * same result; fmaf where the build has the FMA unit (-mfma), the plain form where it would be a libm call */
#ifdef __FMA__
#define DOT_STEP(p, a, w) ((p) = fmaf((a), (w), (p)))
#else
#define DOT_STEP(p, a, w) ((p) += (a) * (w))
#endif

static float LUT[256];

static void lut_init(void)
{
    for (int c = 0; c < 256; c++) {
        const int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
        float v;
        if ((c & 0x7f) == 0x7f) v = 0.0f; /* NaN codes: never produced by the packers */
        else if (e) v = (1.0f + m / 8.0f) * (float)(1 << e) / 128.0f;
        else v = (m / 8.0f) / 64.0f;
        LUT[c] = s ? -v : v;
    }
}

static uint16_t to_bf16(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

int cg_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* qa [M][lda] E4M3, sa [K/128][lds], qw [N][K] E4M3 (N % 4 == 0), sw [ceil(N/128)][K/128] -> cb [M][ldc] bf16.
 * K % 128 == 0. Rows m0 .. m1 - 1 only (a bounded sample of a larger GEMM). threads <= 0: all. */
void cg_gemm(const uint8_t *qa, int lda, const float *sa, int lds, const uint8_t *qw, const float *sw, int N, int K,
             int m0, int m1, uint16_t *cb, int ldc, int threads)
{
    const int KB = K / 128;
    float *wd;

    if (LUT[0x38] == 0.0f) lut_init(); /* 0x38 = 1.0 */
    if (threads <= 0) threads = cg_max_threads();
    wd = (float *)malloc((size_t)N * K * sizeof(float));
    if (!wd) return;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int n = 0; n < N; n++)
        for (int k = 0; k < K; k++) wd[(size_t)n * K + k] = LUT[qw[(size_t)n * K + k]];
#pragma omp parallel num_threads(threads)
    {
        float *ad = (float *)malloc((size_t)128 * K * sizeof(float));
#pragma omp for schedule(dynamic, 1)
        for (int mb = m0; mb < m1; mb += 128) {
            const int mr = m1 - mb < 128 ? m1 - mb : 128;
            for (int i = 0; i < mr; i++)
                for (int k = 0; k < K; k++) ad[(size_t)i * K + k] = LUT[qa[(size_t)(mb + i) * lda + k]];
            for (int n0 = 0; n0 < N; n0 += 4)
                for (int i = 0; i < mr; i += 2) {
                    const int two = i + 1 < mr ? 2 : 1;
                    float acc[2][4] = {{0}};
                    for (int kb = 0; kb < KB; kb++) {
                        float p[2][4][8];
                        const float *a0 = ad + (size_t)i * K, *a1 = ad + (size_t)(i + two - 1) * K;
                        const float *w0 = wd + (size_t)n0 * K;
#ifdef __AVX2__
                        /* the 8 partial sums of each (row, column) as one 8-float vector (GNU vector extension) */
                        typedef float v8 __attribute__((vector_size(32)));
                        v8 v[2][4];
                        for (int r = 0; r < 2; r++)
                            for (int j = 0; j < 4; j++) v[r][j] = (v8){0, 0, 0, 0, 0, 0, 0, 0};
                        for (int k = 128 * kb; k < 128 * kb + 128; k += 8) {
                            v8 x0, x1;
                            memcpy(&x0, a0 + k, 32);
                            memcpy(&x1, a1 + k, 32);
                            for (int j = 0; j < 4; j++) {
                                v8 y;
                                memcpy(&y, w0 + (size_t)j * K + k, 32);
                                for (int l = 0; l < 8; l++) {
                                    DOT_STEP(v[0][j][l], x0[l], y[l]);
                                    DOT_STEP(v[1][j][l], x1[l], y[l]);
                                }
                            }
                        }
                        memcpy(p, v, sizeof(p));
#else
                        memset(p, 0, sizeof(p));
                        for (int k = 128 * kb; k < 128 * kb + 128; k += 8)
                            for (int j = 0; j < 4; j++) {
                                const float *w = w0 + (size_t)j * K + k;
                                for (int l = 0; l < 8; l++) {
                                    DOT_STEP(p[0][j][l], a0[k + l], w[l]);
                                    DOT_STEP(p[1][j][l], a1[k + l], w[l]);
                                }
                            }
#endif
                        for (int r = 0; r < two; r++)
                            for (int j = 0; j < 4; j++) {
                                const float *q = p[r][j];
                                const float part = ((q[0] + q[4]) + (q[2] + q[6])) + ((q[1] + q[5]) + (q[3] + q[7]));
                                const float sc = sa[(size_t)kb * lds + mb + i + r] * sw[(size_t)((n0 + j) / 128) * KB + kb];
                                acc[r][j] = fmaf(part, sc, acc[r][j]);
                            }
                    }
                    for (int r = 0; r < two; r++)
                        for (int j = 0; j < 4; j++) cb[(size_t)(mb + i + r) * ldc + n0 + j] = to_bf16(acc[r][j]);
                }
        }
        free(ad);
    }
    free(wd);
}
