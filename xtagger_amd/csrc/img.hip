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
//   k_img_vpass tmp [S][cw * 4] fp32: output row i over the rect's columns, all RGBX channels (pi_vrow);
//   k_img_hpass one 14-row band of 2 patches per block: each output pixel's B, G, R over its horizontal taps (pi_hrow),
//               staged in shared memory in the operand's own layout and written out as contiguous 16-byte stores.
// Each block builds the tap tables it needs (pi_axis) in shared memory: every tap weight in parallel, each output's sum
// over its taps in the reference's order by one thread.
// A rect whose long side is S skips the resample (pi_idrow): k_img_ident normalises and white-pads the band directly.
#include <pthread.h>

#include "xt_abi.h"
#include "xtag_eva.h"

#define IMG_BAND_P 2                        // patches per band block (2 x 592 halves = 2368 contiguous bytes)
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

// ---- pi_cubic / pi_axis (procimg.h:750-790), built per block in shared memory
__device__ __forceinline__ float img_cubic(float x)
{
    x = x < 0 ? -x : x;
    return x < 1.0f ? (1.5f * x - 2.5f) * x * x + 1.0f : x < 2.0f ? ((-0.5f * x + 2.5f) * x - 4.0f) * x + 2.0f : 0.0f;
}

// One axis: output index i of S over a virtual square of `side` with the content at [off, off + len); the weights
// come out scaled by sc, the constant offset by add (the x axis folds the [-1, 1] normalisation in).
struct ImgGeom {
    float scale, ss, support, sc, add;
    int32_t side, off, end;
};

__device__ __forceinline__ ImgGeom img_geom(uint32_t S, uint32_t side, uint32_t off, uint32_t len, float sc, float add)
{
    ImgGeom g;
    g.scale = (float)side / (float)S;
    const float fs = g.scale > 1.0f ? g.scale : 1.0f;
    g.support = 2.0f * fs;
    g.ss = 1.0f / fs;
    g.sc = sc;
    g.add = add;
    g.side = (int32_t)side;
    g.off = (int32_t)off;
    g.end = (int32_t)(off + len);
    return g;
}

// the taps [lo, hi) of output i and the content part [a, b) of them (pi_axis's integer bounds)
__device__ __forceinline__ void img_bounds(const ImgGeom &g, int32_t i, float &center, int32_t &lo, int32_t &hi,
                                           int32_t &a, int32_t &b)
{
    center = ((float)i + 0.5f) * g.scale;
    lo = (int32_t)(center - g.support + 0.5f);
    hi = (int32_t)(center + g.support + 0.5f);
    lo = lo < 0 ? 0 : lo;
    hi = hi > g.side ? g.side : hi;
    a = lo > g.off ? lo : g.off;
    b = hi < g.end ? hi : g.end;
    b = b < a ? a : b;
}

// Tap tables of `cnt` consecutive outputs i0 .. i0 + cnt - 1 into shared memory: every tap weight in parallel (the same
// float expression as the reference), then one thread per output sums its taps in tap order (the reference's loop),
// then the content taps are scaled. w [cnt][mt] holds the content taps; s, n, k per output. Ends synchronised.
__device__ __forceinline__ void img_taps(const ImgGeom &g, int32_t i0, int32_t cnt, int32_t mt, float *w, int32_t *s,
                                         int32_t *n, float *k, float *sum)
{
    for (int32_t e = threadIdx.x; e < cnt * mt; e += blockDim.x) {
        const int32_t c = e / mt, t = e - c * mt;
        float center;
        int32_t lo, hi, a, b;
        img_bounds(g, i0 + c, center, lo, hi, a, b);
        w[e] = lo + t < hi ? img_cubic(((float)(lo + t) - center + 0.5f) * g.ss) : 0.0f;
    }
    __syncthreads();
    for (int32_t c = threadIdx.x; c < cnt; c += blockDim.x) {
        float center, sm = 0.0f, white = 0.0f;
        int32_t lo, hi, a, b;
        img_bounds(g, i0 + c, center, lo, hi, a, b);
        for (int32_t j = lo; j < hi; j++) {
            const float wt = w[c * mt + (j - lo)];
            sm += wt;
            white += j < a || j >= b ? wt : 0.0f;
        }
        sm = g.sc / sm;
        sum[c] = sm;
        s[c] = a - g.off;
        n[c] = b - a;
        k[c] = 255.0f * white * sm + g.add;
    }
    __syncthreads();
    // content taps to the front of the row, scaled (pi_axis's memmove and wi[j] *= sum), in place: each thread moves
    // the taps of one output so no row is read after another thread overwrote it
    for (int32_t c = threadIdx.x; c < cnt; c += blockDim.x) {
        float center;
        int32_t lo, hi, a, b;
        img_bounds(g, i0 + c, center, lo, hi, a, b);
        for (int32_t q = 0; q < b - a; q++) w[c * mt + q] = w[c * mt + (a - lo) + q] * sum[c];
    }
    __syncthreads();
}

#define IMG_MT_MAX 24                       // taps per output up to a resample factor of 5 (mt = 2 (int)(2 f + 1) + 2)

// ---- pi_vrow (procimg.h:800-836): tmp[i][4 x + c] = k + sum_j w[j] * src(s + j)[x].c, one RGBX pixel per thread;
// block (blockIdx.x, i = blockIdx.y) builds the y tap table of output row i
__global__ void __launch_bounds__(256) k_img_vpass(const uint8_t *__restrict__ src, size_t stride, uint32_t cw,
                                                   uint32_t ch, uint32_t S, uint32_t side, uint32_t mt,
                                                   float4 *__restrict__ tmp)
{
    __shared__ float w[IMG_MT_MAX], sum[1], k[1];
    __shared__ int32_t sn[2];
    const uint32_t i = blockIdx.y, x = blockIdx.x * 256 + threadIdx.x;
    img_taps(img_geom(S, side, (side - ch) >> 1, ch, 1.0f, 0.0f), (int32_t)i, 1, (int32_t)mt, w, sn, sn + 1, k, sum);
    if (x >= cw) return;
    const int32_t s = sn[0], n = sn[1];
    float a0 = k[0], a1 = a0, a2 = a0, a3 = a0;
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

// Band staging: 14 rows x np patches of the operand, [patch][592] halves, pad halves zero; written out with 16-byte
// stores (the band's patches are contiguous in the operand).
__device__ __forceinline__ void img_band_store(uint16_t *band, uint16_t *__restrict__ out, uint32_t S, uint32_t np)
{
    __syncthreads();
    const uint32_t pr = S / 14, p0 = blockIdx.y * pr + blockIdx.x * IMG_BAND_P;
    uint4 *dst = (uint4 *)(out + (size_t)p0 * IMG_PATCH);
    const uint4 *sb = (const uint4 *)band;
    for (uint32_t q = threadIdx.x; q < np * IMG_PATCH / 8; q += blockDim.x) dst[q] = sb[q];
}

// ---- pi_hrow (procimg.h:843-868): band blockIdx.y, patches blockIdx.x * IMG_BAND_P ..; one output pixel per
// thread; the block builds the x tap tables of its 14 IMG_BAND_P columns
__global__ void __launch_bounds__(14 * 14 * IMG_BAND_P) k_img_hpass(const float4 *__restrict__ tmp, uint32_t cw,
                                                                  uint32_t S, uint32_t side, uint32_t mt,
                                                                  uint16_t *__restrict__ out)
{
    __shared__ __attribute__((aligned(16))) uint16_t band[IMG_BAND_P * IMG_PATCH];
    __shared__ float w[14 * IMG_BAND_P * IMG_MT_MAX], k[14 * IMG_BAND_P], sum[14 * IMG_BAND_P];
    __shared__ int32_t ts[14 * IMG_BAND_P], tn[14 * IMG_BAND_P];
    const uint32_t pr = S / 14, pc0 = blockIdx.x * IMG_BAND_P;
    const uint32_t np = pr - pc0 < IMG_BAND_P ? pr - pc0 : IMG_BAND_P;
    if (threadIdx.x < np) *(uint2 *)(band + threadIdx.x * IMG_PATCH + 588) = uint2{0u, 0u};
    img_taps(img_geom(S, side, (side - cw) >> 1, cw, 1.0f / 127.5f, -1.0f), (int32_t)(pc0 * 14), (int32_t)(14 * np),
             (int32_t)mt, w, ts, tn, k, sum);
    const uint32_t e = threadIdx.x;
    if (e < 14 * 14 * np) {
        const uint32_t ky = e / (14 * np), jj = e - ky * 14 * np;   // row in the band, column in the block
        const uint32_t i = blockIdx.y * 14 + ky;
        const int32_t n = tn[jj];
        const float *wj = w + jj * mt;
        const float4 *t = tmp + (size_t)i * cw + ts[jj];
        float r = k[jj], g = r, b = r;
        for (int32_t q = 0; q < n; q++) {
            const float4 v = t[q];
            const float wq = wj[q];
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

// scratch: tmp [S][cw] float4 of the vertical pass
static size_t img_scratch(uint32_t S, uint32_t cw) { return (size_t)S * cw * 16; }

extern "C" size_t eva_img_prep_bytes(uint32_t S, uint32_t max_side)
{
    if (!S) S = EVA_S;
    return img_scratch(S, max_side);
}

// pi_prep with the vertical pass staged in `scratch` (bytes long); what names the entry point in errors
static int img_prep(const char *what, const eva_pyr *p, uint32_t x0, uint32_t y0, uint32_t cw, uint32_t ch, uint32_t S,
                    void *scratch, size_t bytes, void *out, void *stream)
{
    if (!S) S = EVA_S;
    if (!p || !p->nlv || p->nlv > EVA_PYR_LV || !p->lv[0]) return xt_fail(what, "no pyramid");
    if (S % 14 || S > 1008 || !out || ((uintptr_t)out & 15))
        return xt_fail(what, "S must be a multiple of 14 up to 1008; out 16-byte aligned");
    if (!cw || !ch || x0 >= p->lw[0] || y0 >= p->lh[0]) return xt_fail(what, "empty or outside rect");
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
        return xt_check(what);
    }
    const uint32_t mt = img_mt(side, S);
    if (mt > IMG_MT_MAX) return xt_fail(what, "rect more than 5x the model side on its level");
    if (!scratch || bytes < img_scratch(S, cw) || ((uintptr_t)scratch & 15))
        return xt_fail(what, "scratch must be 16-byte aligned and hold S x (rect width on its level) x 16 bytes "
                             "(eva_img_prep_bytes(S, side); EVA_IMG_STATIC_BYTES for eva_img_prep_static)");
    float4 *tmp = (float4 *)scratch;
    hipLaunchKernelGGL(k_img_vpass, dim3((cw + 255) / 256, S), dim3(256), 0, st, src, stride, cw, ch, S, side, mt, tmp);
    hipLaunchKernelGGL(k_img_hpass, bands, dim3(14 * 14 * IMG_BAND_P), 0, st, (const float4 *)tmp, cw, S, side, mt,
                       (uint16_t *)out);
    return xt_check(what);
}

extern "C" int eva_img_prep(const eva_pyr *p, uint32_t x0, uint32_t y0, uint32_t cw, uint32_t ch, uint32_t S,
                            void *scratch, size_t bytes, void *out, void *stream)
{
    return img_prep("eva_img_prep", p, x0, y0, cw, ch, S, scratch, bytes, out, stream);
}

// ---- eva_img_prep without a scratch argument, for callers that cannot allocate. The vertical pass is staged in
// img_static, a file-scope device array (one copy per GPU, held until the process ends). In host code the array's name
// is only a stand-in: its device address on the current GPU comes from hipGetSymbolAddress, taken once per device on
// that device's first call and kept in img_static_dev. Every element the horizontal pass reads was written by the
// vertical pass of the same call, so nothing needs clearing between calls; calls that overlap on one GPU race.
static __device__ __align__(256) uint8_t img_static[EVA_IMG_STATIC_BYTES];
#define IMG_MAX_DEVICES 64
static void *img_static_dev[IMG_MAX_DEVICES];
static pthread_mutex_t img_static_mu = PTHREAD_MUTEX_INITIALIZER;

static void *img_static_addr(int dev)
{
    void *ptr;
    pthread_mutex_lock(&img_static_mu);
    ptr = img_static_dev[dev];
    if (!ptr) {
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(img_static)) != hipSuccess) ptr = NULL;
        img_static_dev[dev] = ptr;
    }
    pthread_mutex_unlock(&img_static_mu);
    return ptr;
}

extern "C" int eva_img_prep_static(const eva_pyr *p, uint32_t x0, uint32_t y0, uint32_t cw, uint32_t ch, uint32_t S,
                                   void *out, void *stream)
{
    int dev;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= IMG_MAX_DEVICES)
        return xt_fail("eva_img_prep_static", "no current device");
    void *ptr = img_static_addr(dev);
    if (!ptr) return xt_fail("eva_img_prep_static", "hipGetSymbolAddress of the static scratch failed");
    return img_prep("eva_img_prep_static", p, x0, y0, cw, ch, S, ptr, EVA_IMG_STATIC_BYTES, out, stream);
}
