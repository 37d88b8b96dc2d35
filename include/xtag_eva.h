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
 * Block scale s = amax / 448 (one IEEE division, correctly rounded), s = 1 for a block with |max| < 2^-116: the
 * reference's per-tensor rule (export_eva.py:64-66) applied per block. Activations q = sat_rne(x * (1/s)) per 1x128
 * block along K, 1/s rounded once (eva.h:408); weights q = sat_rne(w / s) per 128x128 block. Activation scales are
 * stored as planes s[K/128][lds] (lds >= rows); weight scales as s[ceil(N/128)][K/128]; weight rows are padded with
 * zeros to a multiple of 128. Every GEMM role promotes each 128-wide K block's partial sum into an fp32 accumulator,
 * acc = fma(partial, sa * sw, acc), so any finite fp32 scales are honoured (with all scales equal this is the
 * reference's alpha * acc, eva.h:415-418).
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

/* ---- engine (eva.h:109-151) ----
 * Caller-allocated like the reference's eva struct. Callers read nt, nt0 and hpn[buf] (procimg.h:1689, 1981);
 * everything else lives behind impl. */
typedef struct eva_impl eva_impl;
typedef struct {
    uint32_t nt, ntp, nt0;                    /* nt = nt0 tags of the file + extra head rows */
    uint32_t nb;                              /* model inputs per launch */
    uint16_t *hpn[EVA_NBUF];                  /* with extra rows: fp16 head inputs [nb][1024] of each batch */
    float *hout[EVA_NBUF];                    /* sigmoid scores [nb][nt] of each batch */
    eva_impl *impl;
} eva;

/* eva.h:573. Reads the weight blob header and starts the device bring-up on its own thread. The blob is the
 * reference's "EVA2" version-2 file (fp16 block weights, export_eva.py without a calibration file); the bring-up
 * packs every block GEMM weight to E4M3 with 128x128 scales on the GPU (each layer as soon as its bytes are on the
 * device, while the host reads the next), so no calibration pass is needed. pool / poolb: accepted and unused (the
 * reference page-locks the caller's pool in place, eva.h:522; this platform cannot register existing memory, so
 * eva_submit stages inputs in engine-owned pinned memory instead). extra: head rows past the file's tags (tag
 * stealing), written with eva_head_put. Batch EVA_NB. */
int eva_open(eva *e, const char *weights, int device, void *pool, size_t poolb, uint32_t extra);
/* eva_open with the batch (model inputs per launch, 1..EVA_NBMAX) as a runtime parameter */
int eva_open_nb(eva *e, const char *weights, int device, void *pool, size_t poolb, uint32_t extra, uint32_t nb);
/* eva_open_nb with flags. EVA_SPARSE24: the bring-up 2:4-prunes the four layer GEMMs' E4M3 weights (magnitude, as
 * src/tools/prune24.py "mag" does to a v3 blob) and the forward runs them on the sparse matrix cores. No reference
 * counterpart as an API (the reference prunes offline with prune24.py and has no sparse kernel). */
#define EVA_SPARSE24 1u
int eva_open_ex(eva *e, const char *weights, int device, void *pool, size_t poolb, uint32_t extra, uint32_t nb,
                uint32_t flags);
int eva_ready(eva *e);                                              /* eva.h:607 */
int eva_poll(eva *e);                                               /* eva.h:620 */
/* eva.h:627. n <= nb inputs, each an fp16 [1024][592] patch operand (BGR in [-1,1], element c*196 + ky*14 + kx,
 * columns 588..591 zero); buf < EVA_NBUF. The inputs are copied into buf's own pinned staging slot (runs of inputs
 * adjacent in memory in one host copy) before the call returns, so the caller may reuse them at once; the call waits
 * only for buf's previous batch, never for batches on other bufs (up to EVA_NBUF in flight). */
int eva_submit(eva *e, uint32_t buf, uint16_t *const *in, uint32_t n);
int eva_query(eva *e, uint32_t buf);                                /* eva.h:662 */
const float *eva_wait(eva *e, uint32_t buf);                        /* eva.h:667: scores [n][nt] */
/* eva.h:645: head row j, fp16 [1024], and its bias. Stream-ordered: batches submitted after the call see the row; w
 * is copied before the call returns. Only row j is repacked (each head row has its own scales). */
int eva_head_put(eva *e, uint32_t j, const uint16_t *w, float bias);
int eva_head_get(eva *e, uint16_t *w, float *bias);                 /* eva.h:653: the file's nt0 rows */
void eva_close(eva *e);                                             /* eva.h:704 */

/* Resident-input path (no reference counterpart; used by benchmarks): the device input buffer
 * [nb][1024][592] fp16, one forward with no host copies, the device scores [nb][nt] fp32, the engine stream (a
 * forward is complete on it: the stream waits for the second lane), and a blocking wait. Every forward, submitted or
 * resident, runs as two halves at once: inputs 0 .. ceil(nb / 2) - 1 on the engine stream, the rest on a second lane
 * with its own activations, stream and graph. */
void *eva_dev_input(eva *e);
int eva_run(eva *e);
const float *eva_dev_output(eva *e);
void *eva_stream_handle(eva *e);
int eva_sync(eva *e);
/* eva.h:312-338 (eva_profile, built there with EVA_PROF): one direct (non-graph) forward with a GPU event after every
 * op, summed per op kind over the layers and printed to stderr as "prof gpu <op> <ms> <share>"; ms (may be NULL)
 * receives the EVA_PROF_OPS sums in the order eva_profile_opname(0 ..) names them: patch+embed, ln1, qkv, flash, oproj,
 * ln2, fc1, fc2, pool+head (the reference's "stat clear" and "(mlp ln)" ops do not exist here: fc1 writes the LN
 * statistics and fc2 folds the LN). Runs on the device input buffer as it stands, the two halves of the batch one
 * after the other (a graph replay runs them at once). */
#define EVA_PROF_OPS 9
int eva_profile(eva *e, double *ms);
const char *eva_profile_opname(int i);

/* ---- kernel launchers (device pointers; stream = hipStream_t or NULL) ---- */

/* Activation packing (kern_common.cuh:97-128 q2 / st4 / st8h): x [M][ldx], in_kind 0 = bf16, 1 = fp32, 2 = fp16,
 * K % 128 == 0 -> q [M][ldq] E4M3, s [K/128][lds]. */
int eva_k_quant_act(const void *x, int in_kind, int ldx, int M, int K, void *q, int ldq, float *s, int lds,
                    void *stream);
/* Weight packing (export_eva.py:64-66 fp8(), per 128x128 block): w [N][K] fp32 -> q [ceil(N/128)*128][K],
 * s [ceil(N/128)][K/128]. */
int eva_k_quant_w(const float *w, int N, int K, void *q, float *s, void *stream);
/* Encoder check: out[i] = E4M3 of the fp32 with bit pattern first + i (NaN patterns excepted). */
int eva_k_e4m3_bits(uint32_t first, uint32_t count, void *out, void *stream);
/* Block-scale rule check: out[i] = bit pattern of the packers' block scale (which 0: amax / 448 correctly rounded, 1
 * below 2^-116; export_eva.py:64-66 per block) or of its inverse (which 1: 1 / s rounded once; eva.h:408) of the fp32
 * with bit pattern first + i. */
int eva_k_scale_bits(uint32_t first, uint32_t count, int which, void *out, void *stream);
/* Block-scaled GEMM (kern_common.cuh:271-356 gemm8 + alpha epilogue, eva_kernels.cu:134-162):
 * C [M][ldc] = sum_kb sa[kb][m] sw[n/128][kb] sum_k qa[m][k] qw[n][k]; out_kind 0 = bf16 (RNE), 1 = fp32. */
int eva_k_gemm(const void *qa, int lda, const float *sa, int lds, const void *qw, const float *sw, int M, int N, int K,
               void *c, int ldc, int out_kind, void *stream);

/* LayerNorm -> E4M3 (kern_common.cuh:147-186 k_ln): x fp16 [rows][1024] -> q [rows][1024], s [8][lds];
 * eps 1e-6, two-pass mean / variance, y = fma((x - mean) * rstd, gamma, beta). rows <= 2^19, lds >= rows; x, g, b
 * and q 16-byte aligned. */
int eva_k_ln(const void *x, const float *g, const float *b, void *q, float *s, int rows, int lds, void *stream);
/* QKV projection with the attention layouts as its epilogue (eva_kernels.cu:41-114 k_qkv): rows = nb * 1025;
 * w from eva_k_prep_w(perm 1); cs [1024][32][2] RoPE (cos, sin) of patch tokens; q, k bf16 [nb][16][1088][64],
 * vt bf16 [nb][16][64][1088] (padded rows are never written; keep them zero). */
int eva_k_qkv(const void *h8, const float *hs, int lds, const void *w, const float *ws, const float *cs, void *q,
              void *k, void *vt, int rows, void *stream);
/* Attention (kern_common.cuh:403-543 flash8, eva_kernels.cu:116-122 k_flash) -> o8 E4M3 [nb*1025][1024] with 1x128
 * scales os [8][lds]; o32 (may be NULL) receives the fp32 output before packing. */
int eva_k_flash(const void *q, const void *k, const void *vt, void *o8, float *os, int lds, int nb, float *o32,
                void *stream);
/* eva_k_flash over nseq sequences of T tokens, q / k bf16 [nseq][16][TP][64], vt [nseq][16][64][TP] with TP >= T
 * rounded up to 64 (padding rows finite; keys past T are masked): the PixAI engine's windowed (T = 576, 9 windows per
 * image) and global (T = 5184) attention (px_kernels.cu:140-154, k_pflash_w / k_pflash_g), output rows s * T + t. */
int eva_k_flash_seq(const void *q, const void *k, const void *vt, void *o8, float *os, int lds, int nseq, int T, int TP,
                    float *o32, void *stream);
/* Out-projection + residual (eva_kernels.cu:134-162 k_oproj): x fp16 [rows][1024] += a8 . Wo^T */
int eva_k_oproj(const void *a8, const float *as, int lds, const void *w, const float *ws, void *x, int rows,
                void *stream);
/* fc1 + SwiGLU + E4M3 repack + row partials (eva_kernels.cu:211-279 k_fc1): h8 [rows][1024] x W12 [5632][1024]
 * (16-unit g / x chunks) -> m8 [rows][2816] E4M3, ms [22][lds], stat [22][lds][2] = (sum h, sum h^2). The pad units
 * 2730..2815 must have zero weights (they are read as zero from row 5472 on). */
int eva_k_fc1(const void *h8, const float *hs, int lds, const void *w, const float *ws, void *m8, float *ms,
              float *stat, int rows, void *stream);
/* eva_k_fc1 with the reference's per-unit quantization multiplier rs [2816] (eva_kernels.cu:211-279 takes rs: the v3
 * blob's 1 / (adq s~), export_eva.py:144): m8 packs h * rs[unit] with 1x128 scales, stat still sums h itself. */
int eva_k_fc1_rs(const void *h8, const float *hs, int lds, const void *w, const float *ws, void *m8, float *ms,
                 float *stat, const float *rs, int rows, void *stream);
/* fc2 with the MLP LayerNorm folded + residual (eva_kernels.cu:286-334 k_fc2): x += rstd (m8 . W~^T - mean c) + d */
int eva_k_fc2(const void *m8, const float *ms, int lds, const void *w, const float *ws, const float *stat,
              const float *cn, const float *dn, void *x, int rows, void *stream);
/* Tag head (kern_common.cuh:679-727 k_headmv, here an FP8 GEMM): out [nb][nt] = sigmoid(pq . Wh^T + hb). The head
 * rows are packed like activations, each row with its own 1x128 scales (eva_k_quant_act of the fp16 rows: w [nt][1024]
 * E4M3, ws [8][ldw] planes), so rewriting one row (eva_head_put) leaves every other row's codes unchanged. nb <= 128. */
int eva_k_head(const void *pq, const float *ps, int lds, const void *w, const float *ws, int ldw, const float *hb,
               float *out, int nb, int nt, void *stream);
/* Patch embedding + position (eva_kernels.cu:126-130 k_pe, 21-33 k_embed): in fp16 [nb*1024][592], pe fp16
 * [1024][592], pos fp32 [1025][1024] -> x fp16 [nb*1025][1024] */
int eva_k_pe(const void *in, const void *pe, const float *pos, void *x, int nb, void *stream);
/* Mean over patch tokens 1..1024 (eva_kernels.cu:402-431 k_pool): x [nb*1025][1024] -> p fp32 [nb][1024] */
int eva_k_pool(const void *x, float *p, int nb, void *stream);
/* Final LayerNorm (kern_common.cuh:188-192 k_lnh) -> fp16 pn [rows][1024] -> E4M3 q [rows][1024], s [8][lds] */
int eva_k_lnh(const float *p, const float *g, const float *b, void *pn, void *q, float *s, int rows, int lds,
              void *stream);
/* Weight packing from fp16 (export_eva.py:52-119 transforms, per 128x128 block): w16 [n_in][ldw] -> fp32 scratch
 * [n_out][k_out] (zero past n_in / k_in; perm 1 quad-splits the q and k heads of Wqkv: row 16 j + i of a head holds
 * dim 4 i + j; colscale may be NULL) -> q [ceil(n_out/128)*128][k_out], s [ceil(n_out/128)][k_out/128]. */
int eva_k_prep_w(const void *w16, int ldw, int n_in, int k_in, int n_out, int k_out, int perm, const float *colscale,
                 float *scratch, void *q, float *s, void *stream);
/* MLP-LN fold terms (export_eva.py:117-119): c[n] = sum_k dec(q[n][k]) s[n/128][k/128] over the packed W~
 * [1024][2816], d[n] = sum_{k<2730} w2[n][k] beta[k] */
int eva_k_fold_cd(const void *q, const float *s, const void *w2, int ldw2, const float *beta, float *c, float *d,
                  void *stream);
/* v3 blob weights (export_eva.py:64-66, 133-147: E4M3 with one fp32 scale per tensor) to the kernels' layout: E4M3
 * rows w8 [n_in][ldw] -> q [n_out][k_out] (rows >= n_in and columns >= k_in zero; perm 1 quad-splits the q and k heads
 * as eva_k_prep_w), every 128 x 128 block scale s [n_out/128][k_out/128] = scale. */
int eva_k_prep_w8(const void *w8, int ldw, int n_in, int k_in, int n_out, int k_out, int perm, float scale, void *q,
                  float *s, void *stream);
/* c[n] = sum_k dec(q[n][k]) s[n/128][k/128] rs[k] over W~ [1024][2816] with its v3 per-unit multipliers rs (the v3
 * blob's c, export_eva.py:145, recomputed for 2:4-pruned W~) */
int eva_k_fold_c_rs(const void *q, const float *s, const float *rs, float *c, void *stream);

/* ---- 2:4 structured-sparse weights (src/tools/prune24.py:43-56 prunes, mma.sp named at
 * prune24.py:1 is never used there) ---- */
/* In every group of 4 consecutive k of each row of the E4M3 weights w [N][K] (in place), zero the 2 smallest
 * |values| (prune24.py "mag" rule); ties drop the lower k first. K % 4 == 0. */
int eva_k_prune24(void *w, int N, int K, void *stream);
/* Compressed layout of 2:4 weights w [N][K] (N % 16 == 0, K % 128 == 0): vals [N/16][K/128][64][16] (lane l = 16 g
 * + r: row 16 t + r, dense k [128 kb + 32 g, +32), the 2 kept bytes of each group of 4 in k order), idx
 * [N/16][K/128][64] u32 (nibble j = p0 | p1 << 2). bad (may be NULL, device int) counts groups with more than 2
 * nonzero bytes (those pack wrongly). */
int eva_k_pack24(const void *w, int N, int K, void *vals, void *idx, int *bad, void *stream);
/* eva_k_gemm with 2:4-sparse weights (v_smfmac_f32_16x16x128_fp8_fp8): vals, idx from eva_k_pack24, sw the dense
 * weights' 128x128 block scales. N % 16 == 0. */
int eva_k_gemm_sp(const void *qa, int lda, const float *sa, int lds, const void *vals, const void *idx, const float *sw,
                  int M, int N, int K, void *c, int ldc, int out_kind, void *stream);
/* The layer kernels with 2:4-sparse weights (vals, idx of eva_k_pack24 in place of w; same epilogues). */
int eva_k_qkv_sp(const void *h8, const float *hs, int lds, const void *vals, const void *idx, const float *ws,
                 const float *cs, void *q, void *k, void *vt, int rows, void *stream);
int eva_k_oproj_sp(const void *a8, const float *as, int lds, const void *vals, const void *idx, const float *ws,
                   void *x, int rows, void *stream);
int eva_k_fc1_sp(const void *h8, const float *hs, int lds, const void *vals, const void *idx, const float *ws,
                 void *m8, float *ms, float *stat, int rows, void *stream);
int eva_k_fc1_rs_sp(const void *h8, const float *hs, int lds, const void *vals, const void *idx, const float *ws,
                    void *m8, float *ms, float *stat, const float *rs, int rows, void *stream);
int eva_k_fc2_sp(const void *m8, const float *ms, int lds, const void *vals, const void *idx, const float *ws,
                 const float *stat, const float *cn, const float *dn, void *x, int rows, void *stream);

/* ---- patch-operand producer on the GPU (src/core/procimg.h:592-969: pi_row_rgbx, pi_pyramid, pi_level / pi_lsrc,
 * pi_prep for the wd model). A decoded image already in device memory becomes the fp16 patch operand the engine
 * reads (eva_dev_input), bit-identical to the reference's CPU producer. ---- */
#define EVA_PYR_LV 12
typedef struct {                     /* pi_pyr (procimg.h:468-472) with device levels */
    uint8_t *lv[EVA_PYR_LV];         /* RGBX levels; lv[0] (lw[0], lh[0], ls[0]) is the caller's decoded image */
    size_t ls[EVA_PYR_LV];           /* row strides in bytes (multiples of 4) */
    uint32_t lw[EVA_PYR_LV], lh[EVA_PYR_LV], nlv;
} eva_pyr;
/* pi_row_rgbx with alpha (procimg.h:592-630), in place: RGBA -> RGBX over white, X = 255 */
int eva_img_over_white(void *rgba, size_t stride, uint32_t w, uint32_t h, void *stream);
/* Device bytes of levels 1.. of pi_pyramid (procimg.h:665-688) for a w x h image at model side S (0: EVA_S). */
size_t eva_img_pyramid_bytes(uint32_t w, uint32_t h, uint32_t S);
/* pi_pyramid: levels 1.. of p into `levels` (32-byte aligned, eva_img_pyramid_bytes), 2x2 boxes of pi_half
 * (procimg.h:636-661); sets p->nlv and the level fields. */
int eva_img_pyramid(eva_pyr *p, void *levels, size_t bytes, uint32_t S, void *stream);
/* Scratch bytes of eva_img_prep for crops whose long side on the chosen level is at most max_side (4 S - 1 covers
 * every crop of a full pyramid). */
size_t eva_img_prep_bytes(uint32_t S, uint32_t max_side);
/* pi_prep (procimg.h:926-969): the level-0 rect (x0, y0, cw, ch) -> out fp16 [(S/14)^2][592] (EVA_IN halves at
 * S = 448; 16-byte aligned), resampled (bicubic onto the white square, [-1, 1], BGR planes) from the level pi_level
 * picks, or normalised as is when the rect's long side on that level is S. The 4 pad halves of each patch row are 0. */
int eva_img_prep(const eva_pyr *p, uint32_t x0, uint32_t y0, uint32_t cw, uint32_t ch, uint32_t S, void *scratch,
                 size_t bytes, void *out, void *stream);
/* eva_img_prep that allocates nothing and takes no scratch argument. No counterpart in the reference: it is for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops). The vertical pass is staged in a
 * library-owned device array of EVA_IMG_STATIC_BYTES on each GPU it runs on (held until the process ends; its address
 * is looked up on the first call on each device): rects whose chosen level needs more than that (S x rect width on
 * the level x 16 bytes, i.e. the long side on the level below 4 S - 1 at S = 448) fail with -1. All calls on one GPU
 * share the array: calls that overlap in time on that GPU race, so issue them on one stream. */
#define EVA_IMG_STATIC_BYTES ((size_t)448 * (4 * 448 - 1) * 16)
int eva_img_prep_static(const eva_pyr *p, uint32_t x0, uint32_t y0, uint32_t cw, uint32_t ch, uint32_t S, void *out,
                        void *stream);

/* ---- PixAI tagger engine (px.h:110-494): the ViTDet-L forward on the px_k_* kernels below ---- */
#define PX_NB 4                               /* default model inputs per launch (px.h:21; even) */
#define PX_NBUF 4                             /* host output buffers (px.h:28) */
#define PX_T 5184                             /* tokens per 1008^2 input: 72 x 72 patches, window-major */
#define PX_LW 576                             /* tokens per attention window */
#define PX_HID 4736
#define PX_NL 32
#define PX_IN ((size_t)PX_T * EVA_K0P)        /* halves per model input */
/* Caller-allocated like the reference's px struct; callers read nt and hout (px.h:68-88). */
typedef struct px_impl px_impl;
typedef struct {
    uint32_t nt, ntp;                         /* tags of the file; rows of its head (nt rounded up to 8) */
    uint32_t nb;                              /* model inputs per launch */
    float *hout[PX_NBUF];                     /* sigmoid scores [nb][nt] of each batch */
    px_impl *impl;
} px;
/* px.h:357. Reads the "PXAI" header and starts the bring-up on its own thread. The blob is version 2
 * (export_pixai.py without a calibration file: fp16 block weights, packed to E4M3 with 128x128 scales on the GPU at
 * bring-up) or version 3 (with a calibration file: SmoothQuant folds, E4M3 block weights with one scale per tensor
 * from the [32][12] table that leads the blob, rs = 1 / (adq3 s3)); a v3 table entry 0..7 that is not a positive
 * finite scale fails px_open. pool / poolb are accepted and unused (inputs are staged into a pinned slot per buf, as
 * eva_submit). */
int px_open(px *p, const char *weights, int device, void *pool, size_t poolb);
/* px_open with the batch (even, 2..100: token rows stay within the kernels' 2^19) as a runtime parameter */
int px_open_nb(px *p, const char *weights, int device, void *pool, size_t poolb, uint32_t nb);
int px_ready(px *p);                                                /* px.h:388 */
int px_poll(px *p);                                                 /* px.h:400 */
/* px.h:406. n <= nb inputs, each an fp16 [5184][592] patch operand in window-major token order; buf < PX_NBUF. */
int px_submit(px *p, uint32_t buf, uint16_t *const *in, uint32_t n);
int px_query(px *p, uint32_t buf);                                  /* px.h:421 */
const float *px_wait(px *p, uint32_t buf);                          /* px.h:426: scores [n][nt] */
void px_close(px *p);                                               /* px.h:457 */
/* Resident-input path, as eva_dev_input .. eva_sync (no reference counterpart; used by benchmarks and tests). A
 * forward runs as two halves at once, inputs 0 .. nb / 2 - 1 on the engine stream and the rest on a second lane. */
void *px_dev_input(px *p);
int px_run(px *p);
const float *px_dev_output(px *p);
void *px_stream_handle(px *p);
int px_sync(px *p);

/* ---- PixAI tagger (ViTDet-L) block kernels on the same block-scaled main loop (px_kernels.cu) ----
 * Rows are window-major tokens (px_kernels.cu:1-4): sequence s = rows L s .. L s + L - 1 with L = 576 (windowed
 * blocks, 9 windows per image) or 5184 (global blocks, one image); rows <= 2^19. LayerNorm is eva_k_ln, attention
 * eva_k_flash_seq (T = TP = L). */
/* px_kernels.cu:133-138 k_ppe: x fp16 [rows][1024] = f16(in . pe^T), in fp16 [rows][592] patch operands in window-major
 * order, pe fp16 [1024][592]; rows % 128 == 0 (an even batch, px.h:21) */
int px_k_pe(const void *in, const void *pe, void *x, int rows, void *stream);
/* px_kernels.cu:16-50 k_pembed: x = f16(LN_1e-5(x + pos[m % T]) g + b) in place, pos fp32 [T][1024] */
int px_k_pembed(void *x, const float *pos, int T, const float *g, const float *b, int rows, void *stream);
/* px_kernels.cu:54-131 k_pqkv: q, k bf16 [rows/L][16][L][64] = RoPE(h8 . Wqkv^T + b) with table row m % L of
 * cs [L][32][2] on every token, vt bf16 [rows/L][16][64][L] = (h8 . Wv^T + b)^T; w from eva_k_prep_w(perm 1), bias
 * fp32 [3072] in natural order; q rows of w and bias carry log2(e)/8. */
int px_k_qkv(const void *h8, const float *hs, int lds, const void *w, const float *ws, const float *bias,
             const float *cs, int L, void *q, void *k, void *vt, int rows, void *stream);
/* px_kernels.cu:156-190 k_pproj: x fp16 [rows][1024] = x + (a8 . Wo^T + bias) */
int px_k_proj(const void *a8, const float *as, int lds, const void *w, const float *ws, const float *bias, void *x,
              int rows, void *stream);
/* px_kernels.cu:202-241 k_pfc1: m8 E4M3 [rows][4736], ms [37][lds] = block-packed rs * gelu(h8 . W1^T + b1), exact erf
 * GELU; rs fp32 [4736] may be NULL (all ones). */
int px_k_fc1(const void *h8, const float *hs, int lds, const void *w, const float *ws, const float *bias,
             const float *rs, void *m8, float *ms, int rows, void *stream);
/* px_kernels.cu:192-200 k_pfc2: x fp16 [rows][1024] = x + (m8 . W2^T + bias), W2 [1024][4736] */
int px_k_fc2(const void *m8, const float *ms, int lds, const void *w, const float *ws, const float *bias, void *x,
             int rows, void *stream);
/* Attention-pool head (px_kernels.cu:341-503; px.h:170-189), T = 5184 tokens per image, rows = nb * T:
 * px_k_hln = k_phln + k_phscore: y fp16 [rows][1024] = f16(LN_1e-5(x) g + b + hpos[m % T]) (hpos fp16 [T][1024]),
 * s fp32 [rows][16] = U y (U fp32 [16][1024], exp2 domain). rows and T at most 2^20. */
int px_k_hln(const void *x, const float *g, const float *b, const void *hpos, int T, const float *U, void *y, float *s,
             int rows, void *stream);
/* k_phsoft + k_phpool + k_phv (px_kernels.cu:401-503) as three launches, T % 576 == 0 and T <= 9216:
 * px_k_hstat: stat float2 [nb][T/576][16] = per 576-token window and head (max_t s, sum_t 2^(s - max));
 * px_k_hpool: part fp32 [nb][T/288][16][1024] = per 288-token window, sum_t P[b][h][t] y[b][t], with P = f16 softmax
 *   of s over all T tokens (exp2 domain) made from stat; P fp16 [nb][16][T] is also written when not NULL;
 * px_k_hproj: o [nb][1024] = f16(Wv[64 h + n] . pooled[b][h]) as fp32 values (pooled = the nw = T/288 window partials
 *   summed in window order; Wv fp16 [1024][1024]); the tag head follows as eva_k_quant_act(o, fp32) + eva_k_head. */
int px_k_hstat(const float *s, float *stat, int nb, int T, void *stream);
int px_k_hpool(const float *s, const float *stat, const void *y, void *P, float *part, int nb, int T, void *stream);
int px_k_hproj(const float *part, int nw, const void *wv, float *o, int nb, void *stream);
/* g[i] = u[i] Phi(u[i]) for n fp32 values by px_k_fc1's GELU (px_kernels.cu:228-229), for testing its accuracy */
int px_probe_gelu(const float *u, float *g, int n, void *stream);

/* ---- on-box ceilings (no reference counterpart; the roofline fractions use peaks measured on the same GPU) ---- */
/* dense FP8 MFMA: blocks x 256 threads, each wave issuing iters x 8 v_mfma_f32_16x16x128_f8f6f4 on register operands
 * (flops = blocks * 4 * iters * 8 * 65536); out [blocks * 256] keeps the result live */
int eva_probe_mfma_fp8(int blocks, int iters, float *out, void *stream);
/* HBM stream copy of bytes (16-byte multiple) from src to dst */
int eva_probe_copy(const void *src, void *dst, size_t bytes, void *stream);
/* LDS read bandwidth: blocks x 256 threads, each reading iters x 16 x 16 bytes conflict-free from a 64 KB array */
int eva_probe_lds(int blocks, int iters, uint32_t *out, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* XTAG_EVA_H */
