/* xtag_eva.h - C-ABI of libxtag_eva.so: the wd / EVA02-Large tagger engine on one AMD MI355X (gfx950), with
 * block-scaled FP8 (OCP E4M3) GEMMs.
 *
 * Two layers, both plain C (no C++ or torch types):
 *   1. The engine API of the reference's src/engine/eva.h:573-745 (eva_open .. eva_close), same names, signatures,
 *      argument meaning and error behaviour, plus a few resident-input entry points for benchmarks.
 *   2. Kernel launchers, one per reference kernel role (src/engine/eva_kernels.cu, kern_common.cuh), taking device
 *      pointers and a hipStream_t (as void *). The reference launches its kernels by name with cuLaunchKernel
 *      (eva.h:174-176); here each role is an extern "C" host function that adds the block-scale pointers.
 *
 * Errors: every int function returns 0 on success, or -1 after printing "eva: <what>: <reason>" to stderr
 * (eva.h:153-176). eva_wait returns NULL on failure.
 *
 * Numerics (all kernels): E4M3 = OCP FP8 E4M3 "fn", encode round-to-nearest-even saturating to +-448.
 * Block scale s = amax / 448 (IEEE), s = 1 for a block with |max| < 2^-116. Activations q = sat_rne(x * (1/s))
 * per 1x128 block along K; weights q = sat_rne(w / s) per 128x128 block. Activation scales are stored as planes
 * s[K/128][lds] (lds >= rows); weight scales as s[ceil(N/128)][K/128]; weight rows are padded with zeros to a
 * multiple of 128.
 */
#ifndef XTAG_EVA_H
#define XTAG_EVA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- model constants (eva.h:48-69) ---- */
#define EVA_NB 8                              /* default model inputs per launch (eva.h:38-40) */
#define EVA_NBMAX 128                         /* largest batch eva_open_nb accepts */
#define EVA_NBUF 8                            /* host input / output buffers (eva.h:41) */
#define EVA_S 448
#define EVA_D 1024
#define EVA_T 1025
#define EVA_NP 1024
#define EVA_K0P 592
#define EVA_NL 24
#define EVA_NH 16
#define EVA_HID 2730
#define EVA_HIDP 2816                         /* hidden padded to 22 blocks of 128 (reference: 2736) */
#define EVA_IN ((size_t)EVA_NP * EVA_K0P)     /* halves per model input */

/* ---- kernel launchers (device pointers; stream = hipStream_t or NULL) ---- */

/* Activation packing (kern_common.cuh:97-128 q2 / st4 / st8h): x [M][ldx], in_kind 0 = bf16, 1 = fp32,
 * K % 128 == 0 -> q [M][ldq] E4M3, s [K/128][lds]. */
int eva_k_quant_act(const void *x, int in_kind, int ldx, int M, int K, void *q, int ldq, float *s, int lds,
                    void *stream);
/* Weight packing (export_eva.py:64-66 fp8(), per 128x128 block): w [N][K] fp32 -> q [ceil(N/128)*128][K],
 * s [ceil(N/128)][K/128]. */
int eva_k_quant_w(const float *w, int N, int K, void *q, float *s, void *stream);
/* Encoder check: out[i] = E4M3 of the fp32 with bit pattern first + i (NaN patterns excepted). */
int eva_k_e4m3_bits(uint32_t first, uint32_t count, void *out, void *stream);
/* Block-scaled GEMM (kern_common.cuh:271-356 gemm8 + alpha epilogue, eva_kernels.cu:134-162):
 * C [M][ldc] = sum_kb sa[kb][m] sw[n/128][kb] sum_k qa[m][k] qw[n][k]; out_kind 0 = bf16 (RNE), 1 = fp32. */
int eva_k_gemm(const void *qa, int lda, const float *sa, int lds, const void *qw, const float *sw, int M, int N, int K,
               void *c, int ldc, int out_kind, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* XTAG_EVA_H */
