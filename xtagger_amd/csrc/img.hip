// img.hip - the patch-operand producer on the GPU: the reference's pi_ingest / pi_pyramid / pi_prep
// (src/core/procimg.h:592-969) for the wd model, from a decoded RGBA(X) image already in device memory to the fp16
// patch operand [(S/14)^2][592] the engine's input buffer holds (procimg.h:1606-1607), with no host round trip.
//
// Same arithmetic as the reference, element for element: the 2x2 pyramid and alpha-over-white in the same integer
// formulas, the axis weights in the same float operations (built without contraction; divisions IEEE), each output
// one fma per tap in tap order (vertical pass, then horizontal pass over RGBX), clamp to [-1, 1], fp16 by
// round-to-nearest-even. The outputs are therefore bit-identical to the reference's.
//
// Data flow of one crop (eva_img_prep): the host picks the level and the rect on it (pi_level / pi_lsrc, scalar), then
//   k_img_axis  the two axes' tap tables (pi_axis) into the scratch;
//   k_img_vpass tmp [S][cw * 4] fp32: output row i over the rect's columns, all RGBX channels (pi_vrow);
//   k_img_hpass one 14-row band of 8 patches per block: each output pixel's B, G, R over its horizontal taps (pi_hrow),
//               staged in shared memory in the operand's own layout and written out as contiguous 16-byte stores.
// A rect whose long side is S skips the resample (pi_idrow): k_img_ident normalises and white-pads the band directly.
#include "xt_abi.h"
#include "xtag_eva.h"

#define IMG_BAND_P 8                        // patches per k_img_hpass block (8 x 592 halves = 9472 contiguous bytes)
#define IMG_PATCH 592                       // halves per patch row of the operand (588 + 4 zero pad)

// ---- pi_row_rgbx with alpha (procimg.h:592-630): c -> (c a + 255 (255 - a)) / 255 rounded, X = 255, in place
__global__ void __launch_bounds__(256) k_img_over_white(uint8_t *__restrict__ p, size_t stride, uint32_t w, uint32_t h)
{
    const uint32_t x = blockIdx.x * 256 + threadIdx.x, y = blockIdx.y;
    if (x >= w || y >= h) return;
    uint32_t *px = (uint32_t *)(p + (size_t)y * stride) + x;
    const uint32_t v = *px, a = v >> 24, ia = 255u * (255u - a);
    uint32_t o = 0xFF000000u;
#pragma unroll
    for (int c = 0; c < 3; c++) {
        const uint32_t t = ((v >> (8 * c)) & 255u) * a + ia;
        o |= ((t + 128u + ((t + 128u) >> 8)) >> 8) << (8 * c);
    }
    *px = o;
}

// ---- pi_half (procimg.h:636-661): one level of the 2x2 box pyramid, per output pixel and channel
// ve = (a + c + 1) >> 1 over the two rows, then (ve + vo) >> 1 over the two columns
__global__ void __launch_bounds__(256) k_img_half(uint8_t *__restrict__ d, size_t ds, const uint8_t *__restrict__ s,
                                                  size_t ss, uint32_t wn, uint32_t hn)
{
    const uint32_t x = blockIdx.x * 256 + threadIdx.x, y = blockIdx.y;
    if (x >= wn || y >= hn) return;
    const uint32_t *p0 = (const uint32_t *)(s + (size_t)(2 * y) * ss + 8 * (size_t)x);
    const uint32_t *p1 = (const uint32_t *)(s + (size_t)(2 * y + 1) * ss + 8 * (size_t)x);
    const uint2 r0 = {p0[0], p0[1]}, r1 = {p1[0], p1[1]};
    uint32_t o = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t ve = (((r0.x >> (8 * c)) & 255u) + ((r1.x >> (8 * c)) & 255u) + 1u) >> 1;
        const uint32_t vo = (((r0.y >> (8 * c)) & 255u) + ((r1.y >> (8 * c)) & 255u) + 1u) >> 1;
        o |= ((ve + vo) >> 1) << (8 * c);
    }
    *(uint32_t *)(d + (size_t)y * ds + 4 * (size_t)x) = o;
}

// ---- pi_cubic / pi_axis (procimg.h:750-790): one thread per output index of one axis
__device__ __forceinline__ float img_cubic(float x)
{
    x = x < 0 ? -x : x;
    return x < 1.0f ? (1.5f * x - 2.5f) * x * x + 1.0f : x < 2.0f ? ((-0.5f * x + 2.5f) * x - 4.0f) * x + 2.0f : 0.0f;
}

struct ImgAxis {   // one axis' tap table in the scratch
    float *w;      // [S][mt], taps inside the content, scaled by sc / (sum of all taps)
    int32_t *s;    // first content pixel of output i
    int32_t *n;    // content taps of output i
    float *k;      // 255 x (white taps' weight) + add
};

__global__ void __launch_bounds__(256) k_img_axis(ImgAxis ax, ImgAxis ay, uint32_t S, uint32_t side, uint32_t mt,
                                                  uint32_t offx, uint32_t lenx, uint32_t offy, uint32_t leny)
{
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= S) return;
    const bool isx = blockIdx.y == 0;
    const ImgAxis t = isx ? ax : ay;
    const uint32_t off = isx ? offx : offy, len = isx ? lenx : leny;
    const float sc = isx ? 1.0f / 127.5f : 1.0f, add = isx ? -1.0f : 0.0f;
    const float scale = (float)side / (float)S, fs = scale > 1.0f ? scale : 1.0f, support = 2.0f * fs, ss = 1.0f / fs;
    const int32_t end = (int32_t)(off + len);
    const float center = ((float)i + 0.5f) * scale;
    int32_t lo = (int32_t)(center - support + 0.5f), hi = (int32_t)(center + support + 0.5f);
    lo = lo < 0 ? 0 : lo;
    hi = hi > (int32_t)side ? (int32_t)side : hi;
    const int32_t a = lo > (int32_t)off ? lo : (int32_t)off;
    int32_t b = hi < end ? hi : end;
    b = b < a ? a : b;
    float sum = 0.0f, white = 0.0f;
    for (int32_t j = lo; j < hi; j++) {  // every tap, in order: the sums of the reference's single loop
        const float wt = img_cubic(((float)j - center + 0.5f) * ss);
        sum += wt;
        white += j < a || j >= b ? wt : 0.0f;
    }
    sum = sc / sum;
    float *wi = t.w + (size_t)i * mt;
    for (int32_t j = a; j < b; j++) wi[j - a] = img_cubic(((float)j - center + 0.5f) * ss) * sum;
    t.s[i] = a - (int32_t)off;
    t.n[i] = b - a;
    t.k[i] = 255.0f * white * sum + add;
}

// ---- pi_vrow (procimg.h:800-836): tmp[i][4 x + c] = k + sum_j w[j] * src(s + j)[x].c, one RGBX pixel per thread
__global__ void __launch_bounds__(256) k_img_vpass(const uint8_t *__restrict__ src, size_t stride, uint32_t cw,
                                                   ImgAxis ay, uint32_t mt, float4 *__restrict__ tmp)
{
    const uint32_t x = blockIdx.x * 256 + threadIdx.x, i = blockIdx.y;
    if (x >= cw) return;
    const int32_t s = ay.s[i], n = ay.n[i];
    const float k = ay.k[i];
    const float *w = ay.w + (size_t)i * mt;
    float a0 = k, a1 = k, a2 = k, a3 = k;
    const uint8_t *p = src + (size_t)s * stride + 4 * (size_t)x;
    for (int32_t j = 0; j < n; j++, p += stride) {
        const uint32_t v = *(const uint32_t *)p;
        const float wj = w[j];
        a0 = __builtin_fmaf(wj, (float)(v & 255u), a0);
        a1 = __builtin_fmaf(wj, (float)((v >> 8) & 255u), a1);
        a2 = __builtin_fmaf(wj, (float)((v >> 16) & 255u), a2);
        a3 = __builtin_fmaf(wj, (float)(v >> 24), a3);
    }
    tmp[(size_t)i * cw + x] = make_float4(a0, a1, a2, a3);
}

__device__ __forceinline__ uint16_t img_f16(float v)
{
    return __builtin_bit_cast(uint16_t, (_Float16)v);  // v_cvt_f16_f32: round to nearest even
}

// Band staging: 14 rows x IMG_BAND_P patches of the operand, [patch][592] halves, pad halves zero; written out with
// 16-byte stores (the band's patches are contiguous in the operand).
__device__ __forceinline__ void img_band_store(uint16_t *band, uint16_t *__restrict__ out, uint32_t S, uint32_t np)
{
    __syncthreads();
    const uint32_t pr = S / 14, p0 = blockIdx.y * pr + blockIdx.x * IMG_BAND_P;
    uint4 *dst = (uint4 *)(out + (size_t)p0 * IMG_PATCH);
    const uint4 *sb = (const uint4 *)band;
    for (uint32_t q = threadIdx.x; q < np * IMG_PATCH / 8; q += blockDim.x) dst[q] = sb[q];
}

// ---- pi_hrow (procimg.h:843-868): output pixels of band blockIdx.y, patches blockIdx.x * 8 .. + 7
__global__ void __launch_bounds__(256) k_img_hpass(const float4 *__restrict__ tmp, uint32_t cw, ImgAxis ax,
                                                   uint32_t mt, uint32_t S, uint16_t *__restrict__ out)
{
    __shared__ __attribute__((aligned(16))) uint16_t band[IMG_BAND_P * IMG_PATCH];
    const uint32_t pr = S / 14, pc0 = blockIdx.x * IMG_BAND_P;
    const uint32_t np = pr - pc0 < IMG_BAND_P ? pr - pc0 : IMG_BAND_P;
    for (uint32_t q = threadIdx.x; q < np; q += blockDim.x) *(uint2 *)(band + q * IMG_PATCH + 588) = uint2{0u, 0u};
    for (uint32_t e = threadIdx.x; e < 14 * 14 * np; e += blockDim.x) {
        const uint32_t ky = e / (14 * np), jj = e - ky * 14 * np;   // row in the band, column in the block
        const uint32_t i = blockIdx.y * 14 + ky, j = pc0 * 14 + jj;
        const int32_t s = ax.s[j], n = ax.n[j];
        const float k = ax.k[j];
        const float *w = ax.w + (size_t)j * mt;
        const float4 *t = tmp + (size_t)i * cw + s;
        float r = k, g = k, b = k;
        for (int32_t q = 0; q < n; q++) {
            const float4 v = t[q];
            const float wq = w[q];
            r = __builtin_fmaf(wq, v.x, r);
            g = __builtin_fmaf(wq, v.y, g);
            b = __builtin_fmaf(wq, v.z, b);
        }
        uint16_t *o = band + (jj / 14) * IMG_PATCH + ky * 14 + jj % 14;
        o[0] = img_f16(__builtin_fminf(__builtin_fmaxf(b, -1.0f), 1.0f));
        o[196] = img_f16(__builtin_fminf(__builtin_fmaxf(g, -1.0f), 1.0f));
        o[392] = img_f16(__builtin_fminf(__builtin_fmaxf(r, -1.0f), 1.0f));
    }
    img_band_store(band, out, S, np);
}

// ---- pi_idrow (procimg.h:874-902): side == S, the identity: v / 127.5 - 1 as one fma, white (0x3C00) pad
__global__ void __launch_bounds__(256) k_img_ident(const uint8_t *__restrict__ src, size_t stride, uint32_t cw,
                                                   uint32_t ch, uint32_t S, uint16_t *__restrict__ out)
{
    __shared__ __attribute__((aligned(16))) uint16_t band[IMG_BAND_P * IMG_PATCH];
    const uint32_t pr = S / 14, pc0 = blockIdx.x * IMG_BAND_P, ox = (S - cw) >> 1, oy = (S - ch) >> 1;
    const uint32_t np = pr - pc0 < IMG_BAND_P ? pr - pc0 : IMG_BAND_P;
    const float sc = 1.0f / 127.5f;
    for (uint32_t q = threadIdx.x; q < np; q += blockDim.x) *(uint2 *)(band + q * IMG_PATCH + 588) = uint2{0u, 0u};
    for (uint32_t e = threadIdx.x; e < 14 * 14 * np; e += blockDim.x) {
        const uint32_t ky = e / (14 * np), jj = e - ky * 14 * np;
        const uint32_t i = blockIdx.y * 14 + ky, j = pc0 * 14 + jj;
        uint16_t *o = band + (jj / 14) * IMG_PATCH + ky * 14 + jj % 14;
        if (i - oy < ch && j - ox < cw) {
            const uint32_t v = *(const uint32_t *)(src + (size_t)(i - oy) * stride + 4 * (size_t)(j - ox));
            o[0] = img_f16(__builtin_fmaf((float)((v >> 16) & 255u), sc, -1.0f));
            o[196] = img_f16(__builtin_fmaf((float)((v >> 8) & 255u), sc, -1.0f));
            o[392] = img_f16(__builtin_fmaf((float)(v & 255u), sc, -1.0f));
        } else {
            o[0] = o[196] = o[392] = 0x3C00;
        }
    }
    img_band_store(band, out, S, np);
}

// ---------------------------------------------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------------------------------------------
static size_t img_a32(size_t n) { return (n + 31) & ~(size_t)31; }

static uint32_t img_mt(uint32_t side, uint32_t S)  // procimg.h:949
{
    return 2 * (uint32_t)(2.0f * (side > S ? (float)side / (float)S : 1.0f) + 1.0f) + 2;
}

extern "C" int eva_img_over_white(void *rgba, size_t stride, uint32_t w, uint32_t h, void *stream)
{
    if (!rgba || !w || !h || stride < (size_t)w * 4 || (stride & 3) || ((uintptr_t)rgba & 3))
        return xt_fail("eva_img_over_white", "bad image (4-byte aligned rows of w RGBA pixels)");
    hipLaunchKernelGGL(k_img_over_white, dim3((w + 255) / 256, h), dim3(256), 0, (hipStream_t)stream, (uint8_t *)rgba,
                       stride, w, h);
    return xt_check("eva_img_over_white");
}

// pi_pyramid's level sizes (procimg.h:665-681), PI_PYRMIN = 2 S: levels 1.. of p from p->lw[0], p->lh[0]
static uint32_t img_levels(eva_pyr *p, uint32_t S)
{
    uint32_t n;
    for (n = 1; n < EVA_PYR_LV; n++) {
        const uint32_t m = p->lw[n - 1] > p->lh[n - 1] ? p->lw[n - 1] : p->lh[n - 1];
        if ((m >> 1) < 2 * S || p->lw[n - 1] < 2 || p->lh[n - 1] < 2) break;
        p->lw[n] = p->lw[n - 1] >> 1;
        p->lh[n] = p->lh[n - 1] >> 1;
        p->ls[n] = img_a32((size_t)p->lw[n] * 4);
    }
    return n;
}

extern "C" size_t eva_img_pyramid_bytes(uint32_t w, uint32_t h, uint32_t S)
{
    eva_pyr p = {};
    p.lw[0] = w;
    p.lh[0] = h;
    const uint32_t n = img_levels(&p, S ? S : EVA_S);
    size_t total = 0;
    for (uint32_t L = 1; L < n; L++) total += p.ls[L] * p.lh[L];
    return total;
}

extern "C" int eva_img_pyramid(eva_pyr *p, void *levels, size_t bytes, uint32_t S, void *stream)
{
    if (!p || !p->lv[0] || !p->lw[0] || !p->lh[0] || p->ls[0] < (size_t)p->lw[0] * 4 || (p->ls[0] & 3) ||
        ((uintptr_t)p->lv[0] & 3))
        return xt_fail("eva_img_pyramid", "level 0 must be set (lv, lw, lh, ls: 4-byte aligned RGBX rows)");
    if (!S) S = EVA_S;
    const uint32_t n = img_levels(p, S);
    size_t total = 0;
    for (uint32_t L = 1; L < n; L++) total += p->ls[L] * p->lh[L];
    if (n > 1 && (!levels || bytes < total || ((uintptr_t)levels & 31)))
        return xt_fail("eva_img_pyramid", "levels must be 32-byte aligned and hold eva_img_pyramid_bytes()");
    uint8_t *blk = (uint8_t *)levels;
    for (uint32_t L = 1; L < n; L++) {
        p->lv[L] = blk;
        blk += p->ls[L] * p->lh[L];
        hipLaunchKernelGGL(k_img_half, dim3((p->lw[L] + 255) / 256, p->lh[L]), dim3(256), 0, (hipStream_t)stream,
                           p->lv[L], p->ls[L], (const uint8_t *)p->lv[L - 1], p->ls[L - 1], p->lw[L], p->lh[L]);
    }
    for (uint32_t L = n; L < EVA_PYR_LV; L++) {
        p->lv[L] = NULL;
        p->lw[L] = p->lh[L] = 0;
        p->ls[L] = 0;
    }
    p->nlv = n;
    return xt_check("eva_img_pyramid");
}

// scratch: two [S][mt] tables and their s / n / k arrays, then tmp [S][cw] float4
static size_t img_scratch(uint32_t S, uint32_t side, uint32_t cw)
{
    const uint32_t mt = img_mt(side, S);
    return img_a32((size_t)2 * S * mt * 4) + img_a32((size_t)6 * S * 4) + (size_t)S * cw * 16;
}

extern "C" size_t eva_img_prep_bytes(uint32_t S, uint32_t max_side)
{
    if (!S) S = EVA_S;
    return img_scratch(S, max_side, max_side);
}

extern "C" int eva_img_prep(const eva_pyr *p, uint32_t x0, uint32_t y0, uint32_t cw, uint32_t ch, uint32_t S,
                            void *scratch, size_t bytes, void *out, void *stream)
{
    if (!S) S = EVA_S;
    if (!p || !p->nlv || p->nlv > EVA_PYR_LV || !p->lv[0]) return xt_fail("eva_img_prep", "no pyramid");
    if (S % 14 || S > 1008 || !out || ((uintptr_t)out & 15))
        return xt_fail("eva_img_prep", "S must be a multiple of 14 up to 1008; out 16-byte aligned");
    if (!cw || !ch || x0 >= p->lw[0] || y0 >= p->lh[0]) return xt_fail("eva_img_prep", "empty or outside rect");
    // pi_level + pi_lsrc (procimg.h:691-716)
    uint32_t L = 0;
    const uint32_t side0 = cw > ch ? cw : ch;
    while (L + 1 < p->nlv && (side0 >> (L + 1)) >= 2 * S) L++;
    uint32_t x1 = (x0 + cw) >> L, y1 = (y0 + ch) >> L;
    x1 = x1 < p->lw[L] ? x1 : p->lw[L];
    y1 = y1 < p->lh[L] ? y1 : p->lh[L];
    x0 >>= L;
    y0 >>= L;
    x0 = x0 < p->lw[L] ? x0 : p->lw[L] - 1;
    y0 = y0 < p->lh[L] ? y0 : p->lh[L] - 1;
    cw = x1 > x0 ? x1 - x0 : 1;
    ch = y1 > y0 ? y1 - y0 : 1;
    const uint8_t *src = p->lv[L] + (size_t)y0 * p->ls[L] + (size_t)x0 * 4;
    const size_t stride = p->ls[L];
    const uint32_t side = cw > ch ? cw : ch, pr = S / 14;
    const dim3 bands((pr + IMG_BAND_P - 1) / IMG_BAND_P, pr);
    hipStream_t st = (hipStream_t)stream;
    if (side == S) {
        hipLaunchKernelGGL(k_img_ident, bands, dim3(256), 0, st, src, stride, cw, ch, S, (uint16_t *)out);
        return xt_check("eva_img_prep");
    }
    if (!scratch || bytes < img_scratch(S, side, cw) || ((uintptr_t)scratch & 31))
        return xt_fail("eva_img_prep", "scratch must be 32-byte aligned and hold eva_img_prep_bytes(S, side)");
    const uint32_t mt = img_mt(side, S);
    uint8_t *sp = (uint8_t *)scratch;
    ImgAxis ax, ay;
    ax.w = (float *)sp;
    ay.w = ax.w + (size_t)S * mt;
    sp += img_a32((size_t)2 * S * mt * 4);
    ax.s = (int32_t *)sp;
    ax.n = ax.s + S;
    ay.s = ax.n + S;
    ay.n = ay.s + S;
    ax.k = (float *)(ay.n + S);
    ay.k = ax.k + S;
    sp += img_a32((size_t)6 * S * 4);
    float4 *tmp = (float4 *)sp;
    hipLaunchKernelGGL(k_img_axis, dim3((S + 255) / 256, 2), dim3(256), 0, st, ax, ay, S, side, mt, (side - cw) >> 1, cw,
                       (side - ch) >> 1, ch);
    hipLaunchKernelGGL(k_img_vpass, dim3((cw + 255) / 256, S), dim3(256), 0, st, src, stride, cw, ay, mt, tmp);
    hipLaunchKernelGGL(k_img_hpass, bands, dim3(256), 0, st, (const float4 *)tmp, cw, ax, mt, S, (uint16_t *)out);
    return xt_check("eva_img_prep");
}
