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
/* head GEMM with per-row weight scales sw [K/128][ldw] (fp64) */
void xo_gemm_rr_f64_rows(const uint8_t *qa, int lda, const float *sa, int lds, const uint8_t *qw, const float *sw,
                         int ldw, int N, int K, const int *rows, int nrows, double *out);
/* fp32 "repo convention": per K block an fp32 fma chain over 128 exact products, then
 * acc = fma(partial, sa * sw, acc). Rows [m0, m1). Output fp32 [M][ldc] and / or bf16 [M][ldc] (NULL to skip).
 * threads: OpenMP threads (<= 0: all). avx2: 1 = 8-lane AVX2 / FMA kernel, 0 = scalar loop. */
void xo_gemm_bs_f32(const uint8_t *qa, int lda, const float *sa, int lds, const uint8_t *qw, const float *sw, int N,
                    int K, int m0, int m1, float *cf, uint16_t *cb, int ldc, int threads, int avx2);
int xo_max_threads(void);

/* ---- LayerNorm -> E4M3 1x128, the order of the device reduction (kern_common.cuh:147-186 semantics) ---- */
/* x fp16 [M][1024] -> q [M][1024], s [8][lds]; also y fp32 [M][1024] if y != NULL */
void xo_ln_quant(const uint16_t *x, const float *g, const float *b, int M, uint8_t *q, float *s, int lds, float *y);

/* ---- EVA02-L pieces (M = nb * 1025 token rows; Tp = 1088 padded attention rows) ---- */
#define XO_D 1024
#define XO_T 1025
#define XO_TP 1088
#define XO_HID 2730
#define XO_HIDP 2816
/* qkv epilogue (eva_kernels.cu:60-113): acc fp32 [M][3072] natural columns q | k | v (head-major, 64 each; q rows
 * of the weight carry log2(e)/8). RoPE on q, k of patch tokens t >= 1 with pair (2i, 2i+1) and angle
 * cs[(t-1)*32 + i] = (cos, sin) (eva_kernels.cu:74-79, export_eva.py:72-74), then bf16 (RNE).
 * q, k: [nb][16][1088][64]; vt: [nb][16][64][1088] (v transposed). Rows t >= 1025 are not written. */
void xo_qkv_epi(const float *acc, int nb, const float *cs, uint16_t *q, uint16_t *k, uint16_t *vt);
/* softmax attention in fp64 (exp2 domain: scores already carry log2(e)/8), one output row per token:
 * o [nb * 1025][1024] at column h * 64 (flash8's math, kern_common.cuh:403-543, without its E4M3 roundings) */
void xo_attention(const uint16_t *q, const uint16_t *k, const uint16_t *vt, int nb, double *o, int threads);
/* the same for nseq sequences of T tokens padded to TP (q, k [nseq][16][TP][64], vt [nseq][16][64][TP] bf16) ->
 * o [nseq * T][1024]; only queries t % qstep == 0 are computed (others untouched) */
void xo_attention_seq(const uint16_t *q, const uint16_t *k, const uint16_t *vt, int nseq, int T, int TP, int qstep,
                      double *o, int threads);
/* fc1 epilogue (eva_kernels.cu:233-268): acc [M][5632] with g / x interleaved in 16-unit chunks
 * (export_eva.py:60-62) -> h = silu(g) * x, fp32 [M][2816] in unit order; stat [22][M][2] = (sum h, sum h^2) over
 * each 128-unit block. silu(g) = g / (1 + exp(-g)), exact form (the reference's tanh.approx is not restated). */
void xo_fc1_epi(const float *acc, int M, float *h, float *stat);
/* fc2 epilogue with the MLP LayerNorm folded (eva_kernels.cu:300-333, export_eva.py:101-104, 117-119):
 * mean = S / 2730, var = Q / 2730 - mean^2, rstd = 1 / sqrt(var + 1e-6), S, Q summed over the 22 blocks in order;
 * x = f16(x + fma(rstd, acc, fma(-mean * rstd, c, d))). x fp16 [M][1024] in place. */
void xo_fc2_epi(const float *acc, int M, const float *stat, const float *c, const float *d, uint16_t *x);
/* out-projection epilogue (eva_kernels.cu:150-160): x = f16(x + acc) */
void xo_oproj_epi(const float *acc, int M, uint16_t *x);
/* ---- PixAI tagger (ViTDet-L) block epilogues (px_kernels.cu); rows are window-major tokens m = L s + t ---- */
#define XO_PX_HID 4736
/* k_pqkv (px_kernels.cu:82-131): acc fp32 [M][3072] natural columns, f = acc + bias (q's log2(e)/8 is in the weights and
 * bias given), RoPE on every q, k token with pair (2i, 2i+1) and angle cs[(m % L) * 32 + i], bf16 (RNE);
 * q, k [M/L][16][L][64], vt [M/L][16][64][L] */
void xo_px_qkv_epi(const float *acc, int M, int L, const float *bias, const float *cs, uint16_t *q, uint16_t *k,
                   uint16_t *vt);
/* k_pproj / k_pfc2 (px_kernels.cu:170-182): x = f16(x + (acc + bias[n])), x fp16 [M][1024] in place */
void xo_px_res_epi(const float *acc, int M, const float *bias, uint16_t *x);
/* k_pfc1 (px_kernels.cu:222-233): h [M][4736] = (u (0.5 (1 + erff(u 0.70710678)))) rs[n], u = acc + bias[n] (libm erff;
 * rs NULL = no multiply), fp32 */
void xo_px_fc1_epi(const float *acc, int M, const float *bias, const float *rs, float *h);
/* k_ppe (px_kernels.cu:133-138): x [M][1024] = f16(in [M][592] . pe [1024][592]^T) over the 588 real columns, float64 dot */
void xo_px_pe(const uint16_t *in, const uint16_t *pe, int M, uint16_t *x);
/* k_pembed (px_kernels.cu:16-50): y = f16(fma((v - mean) rstd, g, b)), v = x + pos[m % T] in fp32, LayerNorm eps 1e-5 in
 * the device's summation order (as xo_ln_quant) */
void xo_px_pembed(const uint16_t *x, int M, int T, const float *pos, const float *g, const float *b, uint16_t *y);
/* attention-pool head (px_kernels.cu:344-503). k_phln + k_phscore: y = f16(fma((x - mean) rstd, g, b) + hpos[m % T])
 * with the LayerNorm (eps 1e-5, IEEE rstd) in the device's summation order (as xo_ln_quant), s [M][16] = U y in
 * float64 from the fp16 y */
void xo_px_hln(const uint16_t *x, int M, int T, const float *g, const float *b, const uint16_t *hpos, const float *U,
               uint16_t *y, double *s);
/* k_phsoft: P [nb][16][T] = 2^(s - max) / sum over the T tokens of each (image, head), float64 */
void xo_px_hsoft(const float *s, int nb, int T, double *P);
/* k_phpool + k_phv: pooled[b][h] = sum_t P[b][h][t] y[b][t], o [nb][1024] = Wv[64 h + n] . pooled[b][h], float64 from
 * the fp16 P and y */
void xo_px_hpool_hv(const uint16_t *P, const uint16_t *y, int nb, int T, const uint16_t *wv, double *o);
/* patch embedding + position (k_pe + k_embed, eva_kernels.cu:21-33, 126-130): in fp16 [nb*1024][592],
 * pe fp16 [1024][592], pos fp32 [1025][1024] -> x fp16 [nb*1025][1024]; x[b,0] = f16(pos[0]),
 * x[b,1+p] = f16((float)dot + pos[1+p]) with the dot in fp64 */
void xo_embed(const uint16_t *in, const uint16_t *pe, const float *pos, int nb, uint16_t *x);
/* mean over tokens 1..1024 (k_pool, eva_kernels.cu:402-431), tokens summed in order: x [nb*1025][1024] -> p [nb][1024] */
void xo_pool(const uint16_t *x, int nb, float *p);
/* final LayerNorm (k_lnh) -> fp16 pn [nb][1024] -> E4M3 of pn with 1x128 scales q [nb][1024], s [8][lds] */
void xo_lnh(const float *p, const float *g, const float *b, int nb, uint16_t *pn, uint8_t *q, float *s, int lds);
/* MLP-LN fold of fc2 (export_eva.py:101-104, 117-119): w2 fp16 [1024][ldw2] (k < 2730 used), gamma, beta [>=2730]
 * -> wt fp32 [1024][2816] = w2 * gamma (zero past 2730), d[n] = sum_k w2[n][k] * beta[k] (fp32, in k order) */
void xo_fold_w2(const uint16_t *w2, int ldw2, const float *gamma, const float *beta, float *wt, float *d);
/* c[n] = sum_k dec(q[n][k]) * s[n/128][k/128] over [1024][2816] (fp32, in k order) */
void xo_fold_c(const uint8_t *q, const float *s, float *c);

/* ---- 2:4 structured sparsity of the block weights (the 2:4-sparse forward) ---- */
/* 2:4 pruning along K of E4M3 weights (src/tools/prune24.py:43-56): in every group of 4 consecutive k of each row,
 * the 2 lowest scores are zeroed. Score |dec(q)| (the "mag" rule) or, with wanda != 0, |dec(q)| * max_n |dec(q[n][k])|
 * (prune24.py:50). Ties drop the lower k first (prune24.py's argsort order is unspecified for ties).
 * q [N][K] bytes in place, K % 4 == 0. */
void xo_prune24(uint8_t *q, int N, int K, int wanda);
/* Compressed 2:4 layout read by the sparse GEMM. For 16-row tile t and 128-wide K block kb, lane l = 16 g + r
 * (g = 0..3, r = 0..15) holds row 16 t + r, dense k in [128 kb + 32 g, +32) as 8 groups of 4:
 *   vals [N/16][K/128][64][16]: group j's two kept bytes at 2j, 2j + 1, in k order;
 *   idx  [N/16][K/128][64] u32: nibble j = p0 | p1 << 2, the positions (0..3, p0 < p1) of those bytes in the group.
 * Kept positions: the group's nonzero bytes, completed with its lowest-k zero positions. N % 16 == 0, K % 128 == 0.
 * Returns -1 (and packs nothing further) if a group holds more than 2 nonzero bytes. */
int xo_pack24(const uint8_t *q, int N, int K, uint8_t *vals, uint32_t *idx);

/* Full wd forward (eva.h:227-310) from the reference's v2 blob tensors (export_eva.py layout, fp16 block weights,
 * HIDP 2736). Weights are packed here with xo_quant_w exactly as the device does. nl layers (24 for the model);
 * out [nb][nt] sigmoid scores, pn [nb][1024] fp16 head inputs. */
typedef struct {
    const uint16_t *pe;          /* [1024][592] */
    const float *pos, *cs;       /* [1025][1024], [1024][32][2] */
    const float *ln1w[24], *ln1b[24], *ln2w[24], *ln2b[24], *mlnw[24], *mlnb[24];
    const uint16_t *wqkv[24];    /* [3072][1024] */
    const uint16_t *wo[24];      /* [1024][1024] */
    const uint16_t *w12[24];     /* [2*2736][1024], 16-unit g / x chunks */
    const uint16_t *w2[24];      /* [1024][2736] */
    const float *fnw, *fnb;
    const uint16_t *hw;          /* [ntp][1024] */
    const float *hb;             /* [ntp] */
    int nt;
    int sparse;                  /* != 0: the four layer GEMMs' E4M3 weights are 2:4-pruned (xo_prune24, magnitude)
                                    after packing; fc2's fold term c is taken from the pruned W~ */
} xo_model;
int xo_forward(const xo_model *m, const uint16_t *in, int nb, int nl, float *out, uint16_t *pn, int threads);

/* kcheck.c:21-22 LCG (rs = rs * 1664525 + 1013904223): frand() in [-1, 1), and kcheck.c:106-107 E4M3 bytes
 * (top byte of the state, redrawn while NaN or exponent field > 9). *rs is the running state. */
void xo_lcg_frand(uint32_t *rs, size_t n, float *out);
void xo_lcg_e4m3(uint32_t *rs, size_t n, uint8_t *out);

/* ---- patch-operand producer (src/core/procimg.h; xt_img.c) ---- */
/* rows of RGBA -> RGBX over white (pi_row_rgbx with alpha, 592-630) */
void xo_img_over_white(uint8_t *d, size_t ds, const uint8_t *s, size_t ss, uint32_t w, uint32_t h);
/* pyramid level: wn x hn pixels from the level above (pi_half, 636-661) */
void xo_img_half(uint8_t *d, size_t ds, const uint8_t *s, size_t ss, uint32_t wn, uint32_t hn);
uint32_t xo_img_levels(uint32_t w, uint32_t h, uint32_t S, uint32_t *lw, uint32_t *lh); /* pi_pyramid sizes */
uint32_t xo_img_level(uint32_t nlv, uint32_t side, uint32_t S);                          /* pi_level */
void xo_img_lsrc(uint32_t L, const uint32_t *lw, const uint32_t *lh, uint32_t *x0, uint32_t *y0, uint32_t *cw,
                 uint32_t *ch);                                                          /* pi_lsrc */
uint32_t xo_img_mt(uint32_t side, uint32_t S);
void xo_img_axis(uint32_t S, uint32_t side, uint32_t off, uint32_t len, uint32_t mt, float sc, float add, float *w,
                 int32_t *s, int32_t *n, float *k);                                      /* pi_axis */
/* pi_prep (926-969) from the level rect: out [(S/14)^2][592] fp16, BGR planes, white pad */
void xo_img_prep(const uint8_t *src, size_t stride, uint32_t cw, uint32_t ch, uint32_t S, uint16_t *out);

#ifdef __cplusplus
}
#endif
#endif
