/* xt_img.c - CPU restatement of the reference's patch-operand producer (src/core/procimg.h), used ONLY as a test
 * checker and as the CPU baseline of the preprocessing benchmark. The product never links or calls anything here.
 *
 * Scalar C in the reference's arithmetic order: every product-sum is one fmaf per tap in tap order (the reference's
 * _mm256_fmadd_ps / _mm_fmadd_ps per element), weights in plain float operations as written (built with
 * -ffp-contract=off), fp16 by round-to-nearest-even (F16C _MM_FROUND_TO_NEAREST_INT).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "xt_oracle.h"

#define XO_DIV255(x) (((x) + 128u + (((x) + 128u) >> 8)) >> 8) /* procimg.h:592 PI_DIV255 */

/* procimg.h:601-630 pi_row_rgbx with alpha (the scalar tail formula; the AVX2 body computes the same in 16-bit lanes):
 * channel c -> DIV255(c * a + 255 * (255 - a)), X = 255 */
void xo_img_over_white(uint8_t *d, size_t ds, const uint8_t *s, size_t ss, uint32_t w, uint32_t h)
{
    for (uint32_t y = 0; y < h; y++) {
        const uint8_t *sr = s + (size_t)y * ss;
        uint8_t *dr = d + (size_t)y * ds;
        for (uint32_t i = 0; i < w; i++) {
            const uint32_t a = sr[4 * i + 3], ia = 255u * (255u - a);
            dr[4 * i] = (uint8_t)XO_DIV255(sr[4 * i] * a + ia);
            dr[4 * i + 1] = (uint8_t)XO_DIV255(sr[4 * i + 1] * a + ia);
            dr[4 * i + 2] = (uint8_t)XO_DIV255(sr[4 * i + 2] * a + ia);
            dr[4 * i + 3] = 255;
        }
    }
}

/* procimg.h:636-661 pi_half: level L+1 pixel (x, y) from the 2x2 block of level L; rows average rounding up, then the
 * two column averages rounding down (the scalar tail; the AVX2 body is vpavgb then avg - ((a ^ b) & 1)) */
void xo_img_half(uint8_t *d, size_t ds, const uint8_t *s, size_t ss, uint32_t wn, uint32_t hn)
{
    for (uint32_t y = 0; y < hn; y++) {
        const uint8_t *r0 = s + (size_t)(2 * y) * ss, *r1 = r0 + ss;
        uint8_t *dr = d + (size_t)y * ds;
        for (uint32_t x = 0; x < wn; x++)
            for (uint32_t c = 0; c < 4; c++) {
                const uint32_t ve = (r0[8 * x + c] + r1[8 * x + c] + 1u) >> 1;
                const uint32_t vo = (r0[8 * x + 4 + c] + r1[8 * x + 4 + c] + 1u) >> 1;
                dr[4 * x + c] = (uint8_t)((ve + vo) >> 1);
            }
    }
}

/* procimg.h:665-681 pi_pyramid's level sizes (PI_PYRMIN = 2 S, PI_LV = 12): returns the level count, lw/lh [12] */
uint32_t xo_img_levels(uint32_t w, uint32_t h, uint32_t S, uint32_t *lw, uint32_t *lh)
{
    uint32_t n;
    lw[0] = w;
    lh[0] = h;
    for (n = 1; n < 12; n++) {
        const uint32_t m = lw[n - 1] > lh[n - 1] ? lw[n - 1] : lh[n - 1];
        if ((m >> 1) < 2 * S || lw[n - 1] < 2 || lh[n - 1] < 2) break;
        lw[n] = lw[n - 1] >> 1;
        lh[n] = lh[n - 1] >> 1;
    }
    return n;
}

/* procimg.h:691-697 pi_level */
uint32_t xo_img_level(uint32_t nlv, uint32_t side, uint32_t S)
{
    uint32_t L;
    for (L = 0; L + 1 < nlv && (side >> (L + 1)) >= 2 * S; L++)
        ;
    return L;
}

/* procimg.h:700-716 pi_lsrc: the level-0 rect on level L (clipped, at least one pixel) */
void xo_img_lsrc(uint32_t L, const uint32_t *lw, const uint32_t *lh, uint32_t *x0, uint32_t *y0, uint32_t *cw,
                 uint32_t *ch)
{
    uint32_t x1 = (*x0 + *cw) >> L, y1 = (*y0 + *ch) >> L;
    x1 = x1 < lw[L] ? x1 : lw[L];
    y1 = y1 < lh[L] ? y1 : lh[L];
    *x0 >>= L;
    *y0 >>= L;
    *x0 = *x0 < lw[L] ? *x0 : lw[L] - 1;
    *y0 = *y0 < lh[L] ? *y0 : lh[L] - 1;
    *cw = x1 > *x0 ? x1 - *x0 : 1;
    *ch = y1 > *y0 ? y1 - *y0 : 1;
}

/* procimg.h:750-755 pi_cubic (Keys, a = -0.5) */
static float xo_cubic(float x)
{
    x = x < 0 ? -x : x;
    return x < 1.0f ? (1.5f * x - 2.5f) * x * x + 1.0f : x < 2.0f ? ((-0.5f * x + 2.5f) * x - 4.0f) * x + 2.0f : 0.0f;
}

/* procimg.h:949 taps per output */
uint32_t xo_img_mt(uint32_t side, uint32_t S)
{
    return 2 * (uint32_t)(2.0f * (side > S ? (float)side / (float)S : 1.0f) + 1.0f) + 2;
}

/* procimg.h:757-790 pi_axis */
void xo_img_axis(uint32_t S, uint32_t side, uint32_t off, uint32_t len, uint32_t mt, float sc, float add, float *w,
                 int32_t *s, int32_t *n, float *k)
{
    const float scale = (float)side / (float)S, fs = scale > 1.0f ? scale : 1.0f, support = 2.0f * fs, ss = 1.0f / fs;
    const int32_t end = (int32_t)(off + len);
    for (int32_t i = 0; i < (int32_t)S; i++) {
        float *wi = w + (size_t)i * mt, sum = 0.0f, white = 0.0f;
        const float center = ((float)i + 0.5f) * scale;
        int32_t lo = (int32_t)(center - support + 0.5f), hi = (int32_t)(center + support + 0.5f);
        lo = lo < 0 ? 0 : lo;
        hi = hi > (int32_t)side ? (int32_t)side : hi;
        int32_t a = lo > (int32_t)off ? lo : (int32_t)off, b = hi < end ? hi : end;
        b = b < a ? a : b;
        for (int32_t j = lo; j < hi; j++) {
            const float wt = xo_cubic(((float)j - center + 0.5f) * ss);
            sum += wt;
            white += j < a || j >= b ? wt : 0.0f;
            wi[j - lo] = wt;
        }
        memmove(wi, wi + (a - lo), (size_t)(b - a) * sizeof(float));
        sum = sc / sum;
        for (int32_t j = 0; j < b - a; j++) wi[j] *= sum;
        s[i] = a - (int32_t)off;
        n[i] = b - a;
        k[i] = 255.0f * white * sum + add;
    }
}

static inline float xo_clamp1(float v)
{
    v = v > -1.0f ? v : -1.0f; /* _mm_max_ps(acc, -1) */
    return v < 1.0f ? v : 1.0f; /* _mm_min_ps(., 1) */
}

/* patch-operand element of output pixel (i, j), plane p (0 = B, 1 = G, 2 = R): procimg.h:1606-1607 jo[j] and the
 * 14-row bands of pi_prep (926-969): patch (i / 14) * (S / 14) + j / 14, element p * 196 + (i % 14) * 14 + j % 14 */
static inline size_t xo_pix(uint32_t S, uint32_t i, uint32_t j, uint32_t p)
{
    return ((size_t)(i / 14) * (S / 14) + j / 14) * 592 + p * 196 + (i % 14) * 14 + j % 14;
}

/* procimg.h:926-969 pi_prep for the wd model (BGR planes, white pad 0x3C00) from the chosen level's rect: src points at
 * its first pixel (RGBX, rows `stride` bytes apart), cw x ch pixels. out [(S/14)^2][592] fp16; the 4 pad halves of each
 * patch row are written zero. tmp: ceil(cw * 4 / 8) * 8 floats; w scratch: 2 * S * mt floats, 6 * S int32/float. */
void xo_img_prep(const uint8_t *src, size_t stride, uint32_t cw, uint32_t ch, uint32_t S, uint16_t *out)
{
    const uint32_t side = cw > ch ? cw : ch, np = (S / 14) * (S / 14);
    for (size_t q = 0; q < np; q++) memset(out + q * 592 + 588, 0, 8);
    if (side == S) { /* pi_idrow (874-902): the identity, v / 127.5 - 1 as one fma; white pad elsewhere */
        const uint32_t ox = (S - cw) >> 1, oy = (S - ch) >> 1;
        const float sc = 1.0f / 127.5f;
        for (uint32_t i = 0; i < S; i++)
            for (uint32_t j = 0; j < S; j++) {
                const int in = (uint32_t)(i - oy) < ch && j >= ox && j < ox + cw;
                for (uint32_t p = 0; p < 3; p++) {
                    uint16_t h = 0x3C00;
                    if (in) h = xo_f32_to_f16(fmaf((float)src[(size_t)(i - oy) * stride + 4 * (j - ox) + (2 - p)], sc, -1.0f));
                    out[xo_pix(S, i, j, p)] = h;
                }
            }
        return;
    }
    const uint32_t mt = xo_img_mt(side, S), n8 = (cw * 4 + 7) >> 3;
    float *wx = (float *)malloc(sizeof(float) * S * mt), *wy = (float *)malloc(sizeof(float) * S * mt);
    float *kx = (float *)malloc(sizeof(float) * S), *ky = (float *)malloc(sizeof(float) * S);
    int32_t *sx = (int32_t *)malloc(sizeof(int32_t) * S), *nx = (int32_t *)malloc(sizeof(int32_t) * S);
    int32_t *sy = (int32_t *)malloc(sizeof(int32_t) * S), *ny = (int32_t *)malloc(sizeof(int32_t) * S);
    float *tmp = (float *)malloc(sizeof(float) * n8 * 8);
    xo_img_axis(S, side, (side - cw) >> 1, cw, mt, 1.0f / 127.5f, -1.0f, wx, sx, nx, kx);
    xo_img_axis(S, side, (side - ch) >> 1, ch, mt, 1.0f, 0.0f, wy, sy, ny, ky);
    for (uint32_t i = 0; i < S; i++) {
        /* pi_vrow (800-836): tmp[c] = k + sum_j w[j] * row(s + j)[c], over the rect's cw * 4 channel values */
        for (uint32_t c = 0; c < cw * 4; c++) {
            float a = ky[i];
            for (int32_t j = 0; j < ny[i]; j++) a = fmaf(wy[(size_t)i * mt + j], (float)src[(size_t)(sy[i] + j) * stride + c], a);
            tmp[c] = a;
        }
        /* pi_hrow (843-868): per output pixel, the 4 channels of RGBX at once; clamp, fp16, planes B G R */
        for (uint32_t j = 0; j < S; j++)
            for (uint32_t p = 0; p < 3; p++) {
                float a = kx[j];
                for (int32_t q = 0; q < nx[j]; q++) a = fmaf(wx[(size_t)j * mt + q], tmp[4 * (sx[j] + q) + (2 - p)], a);
                out[xo_pix(S, i, j, p)] = xo_f32_to_f16(xo_clamp1(a));
            }
    }
    free(wx);
    free(wy);
    free(kx);
    free(ky);
    free(sx);
    free(nx);
    free(sy);
    free(ny);
    free(tmp);
}
