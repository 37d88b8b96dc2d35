/* xt_oracle.h - CPU restatement of the reference's FP8 / EVA02-L path, used ONLY as a test checker.
 *
 * This is test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 * The product (xtagger_amd/libxtag_eva.so) never links, loads or calls anything here.
 *
 * Conventions (each function names the reference file:line it restates; paths relative to the reference root):
 *   E4M3      OCP FP8 E4M3 ("fn": no inf, 0x7F/0xFF NaN), encode RNE with saturation to +-448
 *             (src/engine/kern_common.cuh:97-100 __NV_SATFINITE; src/tools/export_eva.py:64-66 clip + RNE cast),
 *             decode as src/tools/kcheck.c:25-33.
 *   scales    s = amax / 448 (IEEE, correctly rounded); s = 1 when amax < 2^-116 (zero block).
 *             activations: q = sat_rne(x * (1 / s)), 1/s rounded once per 1x128 block (eva.h:408 + kern_common.cuh:106)
 *             weights:     q = sat_rne(w / s) per 128x128 block (export_eva.py:65)
 *   GEMM      C[m][n] = sum_kb sa[kb][m] * sw[n/128][kb] * sum_{k in kb} qa[m][k] * qw[n][k]
 *             (generalises alpha * acc of eva.h:415-418 / eva_kernels.cu:159 to per-block scales)
 *   layouts   activations [M][lda] bytes, activation scales [K/128][lds] (scale planes, lds >= M),
 *             weights [N][K] bytes, weight scales [ceil(N/128)][K/128].
 */
#ifndef XT_ORACLE_H
#define XT_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar codecs ---- */
uint8_t xo_e4m3_encode(float x);                 /* RNE, saturating to +-448; NaN -> 0x7F | sign */
float xo_e4m3_decode(uint8_t b);                 /* kcheck.c:25-33; 0x7F / 0xFF -> NaN */
void xo_e4m3_encode_n(const float *x, size_t n, uint8_t *out);
void xo_e4m3_encode_bits(uint32_t first, uint32_t count, uint8_t *out, int threads); /* fp32 bit patterns */
uint16_t xo_f32_to_bf16(float x);                /* RNE */
float xo_bf16_to_f32(uint16_t h);
uint16_t xo_f32_to_f16(float x);                 /* RNE, overflow -> inf */
float xo_f16_to_f32(uint16_t h);
float xo_block_scale(float amax);                /* amax / 448, or 1 for a zero block */

/* ---- packing ---- */
/* x fp32 [M][ldx], K % 128 == 0 -> q [M][ldq] bytes, s [K/128][lds] */
void xo_quant_act(const float *x, int M, int K, int ldx, uint8_t *q, int ldq, float *s, int lds);
/* w fp32 [N][K], K % 128 == 0 -> q [ceil(N/128)*128][K] bytes (pad rows zero), s [ceil(N/128)][K/128] */
void xo_quant_w(const float *w, int N, int K, uint8_t *q, float *s);

/* ---- block-scaled GEMM references ---- */
/* fp64 accumulate of the dequantized product, for the listed rows: out [nrows][N] */
void xo_gemm_bs_f64_rows(const uint8_t *qa, int lda, const float *sa, int lds, const uint8_t *qw, const float *sw,
                         int N, int K, const int *rows, int nrows, double *out);
/* fp32 "repo convention": per K block an fp32 fma chain over 128 exact products, then
 * acc = fma(partial, sa * sw, acc). Rows [m0, m1). Output fp32 [M][ldc] and / or bf16 [M][ldc] (NULL to skip).
 * threads: OpenMP threads (<= 0: all). avx2: 1 = 8-lane AVX2 / FMA kernel, 0 = scalar loop. */
void xo_gemm_bs_f32(const uint8_t *qa, int lda, const float *sa, int lds, const uint8_t *qw, const float *sw, int N,
                    int K, int m0, int m1, float *cf, uint16_t *cb, int ldc, int threads, int avx2);
int xo_max_threads(void);

/* ---- LayerNorm -> E4M3 1x128, the order of the device reduction (kern_common.cuh:147-186 semantics) ---- */
/* x fp16 [M][1024] -> q [M][1024], s [8][lds]; also y fp32 [M][1024] if y != NULL */
void xo_ln_quant(const uint16_t *x, const float *g, const float *b, int M, uint8_t *q, float *s, int lds, float *y);

/* kcheck.c:21-22 LCG (rs = rs * 1664525 + 1013904223): frand() in [-1, 1), and kcheck.c:106-107 E4M3 bytes
 * (top byte of the state, redrawn while NaN or exponent field > 9). *rs is the running state. */
void xo_lcg_frand(uint32_t *rs, size_t n, float *out);
void xo_lcg_e4m3(uint32_t *rs, size_t n, uint8_t *out);

#ifdef __cplusplus
}
#endif
#endif
