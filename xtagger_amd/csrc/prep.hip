// prep.hip - weight preparation at bring-up: the reference's v2 fp16 block weights (export_eva.py layout) become
// E4M3 with 128x128 fp32 scales on the GPU, with the transforms the kernels expect:
//  - q and k rows of Wqkv quad-split per head: physical column c = 16 j + i of a head holds dim 4 i + j, so a lane
//    of k_qkv holds dims 4 i .. 4 i + 3, two whole rotary pairs (eva_kernels.cu:74-79), and stores them as 8 bytes;
//    quantization blocks are 128 rows = 2 heads, so the split never moves a row across a block (same scales as the
//    natural order);
//  - fc1 rows re-padded from 2 x 2736 to 2 x 2816 units (the 16-unit g / x chunks of export_eva.py:60-62 are
//    chunk-major, so that is a zero tail);
//  - the MLP LayerNorm folded into fc2 (export_eva.py:101-104, 117-119): W~ = W2 diag(gamma), c = W~ 1 from the
//    packed W~ (dequantized, export_eva.py:118), d = W2 beta;
//  - the head (fp16, kept as the master for eva_head_put) packed per 128-row block.
#include "xt_abi.h"
#include "xt_common.h"

extern "C" int eva_k_quant_w(const float *w, int N, int K, void *q, float *s, void *stream);

// fp16 [n_in][ldw] -> fp32 [n_out][k_out]: rows >= n_in and columns >= k_in are zero; perm 1 quad-splits the q and
// k heads (rows < 2048); colscale (may be NULL) multiplies column k (one rounding).
__global__ void __launch_bounds__(256) k_prep_f32(const uint16_t *__restrict__ w, int ldw, int n_in, int k_in,
                                                  int n_out, int k_out, int perm, const float *__restrict__ colscale,
                                                  float *__restrict__ out)
{
    const long total = (long)n_out * k_out;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
        const int r = (int)(i / k_out), c = (int)(i - (long)r * k_out);
        int src = r;
        if (perm == 1 && r < 2 * XT_D) {
            const int hd = r & ~63, pc = r & 63, j = pc >> 4, ii = pc & 15;
            src = hd + 4 * ii + j;
        }
        float v = 0.f;
        if (src < n_in && c < k_in) {
            v = h2f(w[(size_t)src * ldw + c]);
            if (colscale) v = v * colscale[c];
        }
        out[i] = v;
    }
}

// decoded E4M3 value (kcheck.c:25-33)
__device__ __forceinline__ float e4_dec(uint8_t b)
{
    const int e = (b >> 3) & 15, m = b & 7;
    const float v = e ? __builtin_ldexpf(1.0f + m * 0.125f, e - 7) : __builtin_ldexpf(m * 0.125f, -6);
    return (b & 0x80) ? -v : v;
}

// c[n] = sum_k dec(q[n][k]) s[n/128][k/128] over [1024][2816], d[n] = sum_{k < 2730} w2[n][k] beta[k]; one thread
// per row, k in order (fma chains).
__global__ void __launch_bounds__(256) k_fold_cd(const uint8_t *__restrict__ q, const float *__restrict__ s,
                                                 const uint16_t *__restrict__ w2, int ldw2,
                                                 const float *__restrict__ beta, float *__restrict__ c,
                                                 float *__restrict__ d)
{
    const int n = blockIdx.x * 256 + threadIdx.x;
    if (n >= XT_D) return;
    float cc = 0.f, dd = 0.f;
    for (int k = 0; k < XT_HIDP; k++) {
        cc = __builtin_fmaf(e4_dec(q[(size_t)n * XT_HIDP + k]), s[(size_t)(n >> 7) * (XT_HIDP / 128) + (k >> 7)], cc);
        if (k < XT_HID) dd = __builtin_fmaf(h2f(w2[(size_t)n * ldw2 + k]), beta[k], dd);
    }
    c[n] = cc;
    d[n] = dd;
}

extern "C" int eva_k_prep_w(const void *w16, int ldw, int n_in, int k_in, int n_out, int k_out, int perm,
                            const float *colscale, float *scratch, void *q, float *s, void *stream)
{
    if (n_in < 0 || n_in > n_out || k_in > k_out || ldw < k_in || k_out % 128 || n_out <= 0 || (perm != 0 && perm != 1))
        return xt_fail("eva_k_prep_w", "bad shape (n_in <= n_out, k_in <= k_out <= ldw, k_out % 128 == 0)");
    const long total = (long)n_out * k_out;
    long blocks = (total + 255) / 256;
    if (blocks > 65535) blocks = 65535;
    hipLaunchKernelGGL(k_prep_f32, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (const uint16_t *)w16, ldw,
                       n_in, k_in, n_out, k_out, perm, colscale, scratch);
    if (xt_check("eva_k_prep_w")) return -1;
    return eva_k_quant_w(scratch, n_out, k_out, q, s, stream);
}

extern "C" int eva_k_fold_cd(const void *q, const float *s, const void *w2, int ldw2, const float *beta, float *c,
                             float *d, void *stream)
{
    if (ldw2 < XT_HID) return xt_fail("eva_k_fold_cd", "ldw2 must be >= 2730");
    hipLaunchKernelGGL(k_fold_cd, dim3(XT_D / 256), dim3(256), 0, (hipStream_t)stream, (const uint8_t *)q, s,
                       (const uint16_t *)w2, ldw2, beta, c, d);
    return xt_check("eva_k_fold_cd");
}

// v3 blob weights: E4M3 bytes [n_in][ldw] -> q [n_out][k_out] (zero past n_in / k_in, perm 1 as k_prep_f32), one
// 32-bit word of four bytes per thread
__global__ void __launch_bounds__(256) k_prep_w8(const uint8_t *__restrict__ w, int ldw, int n_in, int k_in, int n_out,
                                                 int k_out, int perm, uint8_t *__restrict__ q)
{
    const long total = (long)n_out * (k_out / 4);
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
        const int r = (int)(i / (k_out / 4)), c = 4 * (int)(i - (long)r * (k_out / 4));
        int src = r;
        if (perm == 1 && r < 2 * XT_D) {
            const int hd = r & ~63, pc = r & 63, j = pc >> 4, ii = pc & 15;
            src = hd + 4 * ii + j;
        }
        uint32_t v = 0;
        if (src < n_in)
            for (int b = 0; b < 4; b++)
                if (c + b < k_in) v |= (uint32_t)w[(size_t)src * ldw + c + b] << (8 * b);
        *(uint32_t *)(q + (size_t)r * k_out + c) = v;
    }
}

__global__ void __launch_bounds__(256) k_fill(float *__restrict__ p, int n, float v)
{
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = v;
}

// c[n] = sum_k dec(q[n][k]) s[n/128][k/128] rs[k], one thread per row, k in order (fma chains)
__global__ void __launch_bounds__(256) k_fold_c_rs(const uint8_t *__restrict__ q, const float *__restrict__ s,
                                                   const float *__restrict__ rs, float *__restrict__ c)
{
    const int n = blockIdx.x * 256 + threadIdx.x;
    if (n >= XT_D) return;
    float cc = 0.f;
    for (int k = 0; k < XT_HIDP; k++)
        cc = __builtin_fmaf(e4_dec(q[(size_t)n * XT_HIDP + k]) * s[(size_t)(n >> 7) * (XT_HIDP / 128) + (k >> 7)], rs[k], cc);
    c[n] = cc;
}

extern "C" int eva_k_prep_w8(const void *w8, int ldw, int n_in, int k_in, int n_out, int k_out, int perm, float scale,
                             void *q, float *s, void *stream)
{
    if (n_in < 0 || n_in > n_out || k_in > k_out || ldw < k_in || k_out % 128 || n_out % 128 || n_out <= 0 ||
        (perm != 0 && perm != 1) || !(scale > 0.f))
        return xt_fail("eva_k_prep_w8", "bad shape or scale (n_in <= n_out, k_in <= k_out <= ldw, n_out and k_out "
                                        "multiples of 128, scale > 0)");
    if ((uintptr_t)q & 3) return xt_fail("eva_k_prep_w8", "q must be 4-byte aligned");
    const long total = (long)n_out * (k_out / 4);
    long blocks = (total + 255) / 256;
    if (blocks > 65535) blocks = 65535;
    hipLaunchKernelGGL(k_prep_w8, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (const uint8_t *)w8, ldw,
                       n_in, k_in, n_out, k_out, perm, (uint8_t *)q);
    if (xt_check("eva_k_prep_w8")) return -1;
    const int ns = (n_out / 128) * (k_out / 128);
    hipLaunchKernelGGL(k_fill, dim3((ns + 255) / 256), dim3(256), 0, (hipStream_t)stream, s, ns, scale);
    return xt_check("eva_k_prep_w8");
}

extern "C" int eva_k_fold_c_rs(const void *q, const float *s, const float *rs, float *c, void *stream)
{
    hipLaunchKernelGGL(k_fold_c_rs, dim3(XT_D / 256), dim3(256), 0, (hipStream_t)stream, (const uint8_t *)q, s, rs, c);
    return xt_check("eva_k_fold_c_rs");
}

