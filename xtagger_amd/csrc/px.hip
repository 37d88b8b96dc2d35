// px.hip - the ViTDet-L (PixAI tagger) block GEMMs on the block-scaled main loop, with the epilogues of
// src/engine/px_kernels.cu: k_pqkv (54-131, bias + RoPE at table row m % L + the attention layouts), k_pproj / k_pfc2
// (156-200, residual + bias) and k_pfc1 (202-241, bias + exact-erf GELU + per-unit multiplier, packed to E4M3).
//
// Tokens are window-major for the whole network (px_kernels.cu:1-4): image b's 72 x 72 patches are 9 windows of
// 24 x 24, window w = rows 5184 b + 576 w .. + 575. A windowed block's attention runs over sequences of L = 576
// rows, a global block's over L = 5184; both are row m = L s + t of sequence s, token t, so only L differs.
// Activations E4M3 [rows][K] with 1x128 scale planes [K/128][lds]; residual x fp16 [rows][1024]; the reference's
// per-tensor alpha and static quantization scales are the block scales here.
#include "layer_core.h"

#define PX_HID 4736  // MLP hidden units (37 blocks of 128)

typedef float v2f __attribute__((ext_vector_type(2)));

// GELU with the exact normal CDF, u Phi(u) (px_kernels.cu:228-229 computes Phi as 0.5 (1 + erf(u / sqrt 2))), branch
// free: with t = |u|, Phi(-t) = 2^Q(t), Q(t) = -t^2 / (2 ln 2) + R(t), and R a degree-12 polynomial in s = t / 4 - 1
// fitted to log2 Phi(-t) + t^2 / (2 ln 2) on [0, 8] (Chebyshev least squares reweighted toward minimax: |R error|
// 1.6e-7); then Phi(u) = 2^Q for u < 0 and 1 - 2^Q otherwise, with no cancellation on either side. In fp32 against
// float64: Phi(-t) within 2.9e-6 relative on [0, 8] (the rounding of Q), 1 - Phi(-t) within 1.7e-7 absolute. Past
// t = 8 R is held at R(8): Phi(-t) < 6.3e-16 there and comes out within a factor t / 8. One v_exp_f32 and 17 fp32
// operations per unit, where erff takes two divergent branches.
__device__ __forceinline__ float gelu_erf(float u)
{
    const float t = __builtin_fabsf(u), s = __builtin_fmaf(__builtin_fminf(t, 8.0f), 0.25f, -1.0f);
    float r = -1.352992957e-03f;
    r = __builtin_fmaf(r, s, 2.075498225e-03f);
    r = __builtin_fmaf(r, s, 1.706041396e-03f);
    r = __builtin_fmaf(r, s, -4.959797952e-03f);
    r = __builtin_fmaf(r, s, 6.737539079e-03f);
    r = __builtin_fmaf(r, s, -1.677700505e-02f);
    r = __builtin_fmaf(r, s, 3.916485980e-02f);
    r = __builtin_fmaf(r, s, -7.741049677e-02f);
    r = __builtin_fmaf(r, s, 1.462343782e-01f);
    r = __builtin_fmaf(r, s, -2.747326195e-01f);
    r = __builtin_fmaf(r, s, 5.386815071e-01f);
    r = __builtin_fmaf(r, s, -1.301931143e+00f);
    r = __builtin_fmaf(r, s, -3.404906750e+00f);
    const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(-0.72134752f, t * t, r));  // Phi(-t)
    return u * (u < 0.0f ? e : 1.0f - e);
}

// ---------------------------------------------------------------------------------------------------------------
// k_px_qkv: h8 [rows][1024] x Wqkv [3072][1024] + bias -> q, k bf16 [S][16][L][64] (RoPE on every token with table
// row t = m % L, cs [L][32] (cos, sin) of pair i = dims 2i, 2i+1), vt bf16 [S][16][64][L]; rows = S L. Weight rows of
// q and k are pair-split as for the wd model (column tile 2p of a head holds dims 2i, tile 2p+1 dims 2i+1 of pair
// i = 16p + (lane & 15)); the bias stays in natural order. q rows of W and of the bias carry log2(e)/8 (the
// reference's cq, px_kernels.cu:84).
// ---------------------------------------------------------------------------------------------------------------
template <bool SP>
__global__ void __launch_bounds__(LayerCfg::NT) k_px_qkv(const uint8_t *__restrict__ h8, const float *__restrict__ hs,
                                                        int lds, const uint8_t *__restrict__ w,
                                                        const uint32_t *__restrict__ wx, const float *__restrict__ ws,
                                                        const float *__restrict__ bias, const float *__restrict__ cs,
                                                        int L, uint16_t *__restrict__ q, uint16_t *__restrict__ k,
                                                        uint16_t *__restrict__ vt, int rows)
{
    using C = LayerCfg;
    __shared__ __attribute__((aligned(16))) uint8_t smem[LAYER_SMEM];
    v4f acc[C::TM][C::TN];
    int m0, n0, wm0, wn0;
    layer_tile<C>(rows, 3 * XT_D, m0, n0);
    args_resident(bias, cs, q, k, vt, L, lds, rows);
    layer_mainloop<C, SP>(h8, XT_D, hs, lds, w, wx, ws, rows, 3 * XT_D, XT_D, m0, n0, smem, acc);
    bs_wave_origin<C>(wm0, wn0);
    const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    const int part = n0 >> 10, head0 = ((n0 & 1023) + wn0) >> 6;
    if (part < 2) {
        // every (cos, sin) pair of the tile is loaded before the first store. Stores go through a descriptor that ends
        // at sequence S: rows past `rows` map to sequence S or later and are dropped without a branch.
        const __amdgpu_buffer_rsrc_t rc = buf_rsrc(cs, (uint32_t)L * 32u * 8u);
        const __amdgpu_buffer_rsrc_t rd = buf_rsrc(part ? k : q, (uint32_t)rows * XT_D * 2u);
        v2f bq[2][2];
#pragma unroll
        for (int hh = 0; hh < 2; hh++)
#pragma unroll
            for (int p = 0; p < 2; p++)
                bq[hh][p] = *(const v2f *)(bias + part * XT_D + (head0 + hh) * XT_HD + 2 * (16 * p + c16));
        v2f rot[C::TM][4][2];
        uint32_t base[C::TM][4];  // element offset of (sequence, head head0, token), dims 0
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm0 + 16 * i + 4 * g + r, s = m / L, t = m - s * L;
                base[i][r] = ((uint32_t)(s * XT_NH + head0) * (uint32_t)L + (uint32_t)t) * XT_HD;
#pragma unroll
                for (int p = 0; p < 2; p++)
                    rot[i][r][p] = __builtin_bit_cast(
                        v2f, __builtin_amdgcn_raw_buffer_load_b64(rc, (int)(((uint32_t)t * 32u + 16 * p + c16) * 8u), 0, 0));
            }
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int hh = 0; hh < 2; hh++)
#pragma unroll
                    for (int p = 0; p < 2; p++) {
                        const int pi = 16 * p + c16;
                        const float f0 = acc[i][4 * hh + 2 * p][r] + bq[hh][p].x;
                        const float f1 = acc[i][4 * hh + 2 * p + 1][r] + bq[hh][p].y;
                        const v2f a = rot[i][r][p];
                        const float g0 = f0 * a.x - f1 * a.y, g1 = f1 * a.x + f0 * a.y;
                        const uint32_t off = (base[i][r] + (uint32_t)(hh * L * XT_HD + 2 * pi)) * 2u;
                        __builtin_amdgcn_raw_buffer_store_b32(pk_bf16(g0, g1), rd, (int)off, 0, 0);
                    }
        return;
    }
    // v (+ bias): transpose the wave's 64 rows x 128 dims (two heads) through LDS, then lanes walk rows (consecutive
    // tokens of one sequence: L is a multiple of 64 and the wave's 64 rows start on a multiple of 64)
    float bv[C::TN];
#pragma unroll
    for (int j = 0; j < C::TN; j++) bv[j] = bias[n0 + wn0 + 16 * j + c16];
    uint16_t *tr = (uint16_t *)(smem + (threadIdx.x >> 6) * 128 * 66 * 2);  // [128 dims][66] bf16, padded rows
#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int j = 0; j < C::TN; j++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                tr[(16 * j + c16) * 66 + 16 * i + 4 * g + r] = (uint16_t)pk_bf16(acc[i][j][r] + bv[j], 0.f);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const int m = m0 + wm0 + lane;
    if (m < rows) {
        const int s = m / L, t = m - s * L;
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            uint16_t *dst = vt + ((size_t)s * XT_NH + head0 + hh) * XT_HD * L + t;
#pragma unroll 8
            for (int d = 0; d < XT_HD; d++) dst[(size_t)d * L] = tr[(64 * hh + d) * 66 + lane];
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// k_px_res: x [rows][1024] = f16(x + (a8 . W^T + bias)), K = 1024 (attention out-projection, k_pproj) or 4736 (fc2,
// k_pfc2). The reference rounds (x + alpha acc) + b in fp32 (px_kernels.cu:178); here acc + b is formed first: the
// two orders differ by at most one fp32 rounding before the fp16 store.
// ---------------------------------------------------------------------------------------------------------------
struct PxAddBias {
    float b[LayerCfg::TN];  // the lane's column biases, held by value (registers)
    __device__ __forceinline__ float operator()(int, int j, int, float v) const { return v + b[j]; }
};

template <bool SP, int K>
__global__ void __launch_bounds__(LayerCfg::NT) k_px_res(const uint8_t *__restrict__ a8, const float *__restrict__ as,
                                                        int lds, const uint8_t *__restrict__ w,
                                                        const uint32_t *__restrict__ wx, const float *__restrict__ ws,
                                                        const float *__restrict__ bias, uint16_t *__restrict__ x,
                                                        int rows)
{
    using C = LayerCfg;
    __shared__ __attribute__((aligned(16))) uint8_t smem[LAYER_SMEM];
    v4f acc[C::TM][C::TN];
    int m0, n0, wm0, wn0;
    layer_tile<C>(rows, XT_D, m0, n0);
    args_resident(bias, x, lds, rows);
    layer_mainloop<C, SP>(a8, K, as, lds, w, wx, ws, rows, XT_D, K, m0, n0, smem, acc);
    bs_wave_origin<C>(wm0, wn0);
    const int c16 = threadIdx.x & 15;
    PxAddBias f;
#pragma unroll
    for (int j = 0; j < C::TN; j++) f.b[j] = bias[n0 + wn0 + 16 * j + c16];
    residual_add<C>(smem, acc, x, m0 + wm0, n0 + wn0, rows, f);
}

// ---------------------------------------------------------------------------------------------------------------
// k_px_fc1: h8 [rows][1024] x W1 [4736][1024] -> h = rs (gelu(acc + b1)), gelu(u) = u Phi(u) (exact normal CDF,
// px_kernels.cu:228-231, by gelu_erf; rs may be NULL = 1), packed to m8 [rows][4736] E4M3 with 1x128 scales
// ms [37][lds]. A wave's 128 columns are one scale block: each row's |max| meets in a 16-lane DPP reduction, the
// values are scaled in registers, parked in the wave's own LDS slice 64 columns at a time and stored 8 consecutive
// bytes per lane (8 rows of 64 bytes per wave instruction). The second half of the last column tile lies past
// unit 4736 and stores nothing.
// ---------------------------------------------------------------------------------------------------------------
template <bool SP, bool RS>
__global__ void __launch_bounds__(LayerCfg::NT) k_px_fc1(const uint8_t *__restrict__ h8, const float *__restrict__ hs,
                                                        int lds, const uint8_t *__restrict__ w,
                                                        const uint32_t *__restrict__ wx, const float *__restrict__ ws,
                                                        const float *__restrict__ bias, const float *__restrict__ rs,
                                                        uint8_t *__restrict__ m8, float *__restrict__ ms, int rows)
{
    using C = LayerCfg;
    static_assert(C::TM == 4 && C::TN == 8 && C::WN == 128, "a wave tile is 64 rows x one 128-unit scale block");
    __shared__ __attribute__((aligned(16))) uint8_t smem[LAYER_SMEM];
    v4f acc[C::TM][C::TN];
    int m0, n0, wm0, wn0;
    layer_tile<C>(rows, PX_HID, m0, n0);
    args_resident(bias, rs, m8, ms, lds, rows);
    layer_mainloop<C, SP>(h8, XT_D, hs, lds, w, wx, ws, rows, PX_HID, XT_D, m0, n0, smem, acc);
    bs_wave_origin<C>(wm0, wn0);
    const int blk = (n0 + wn0) >> 7;
    if (blk >= PX_HID / 128) return;  // no block barrier follows: the epilogue uses the wave's own slice only
    const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    float bj[C::TN], rj[C::TN];
#pragma unroll
    for (int j = 0; j < C::TN; j++) {
        const int u = 128 * blk + 16 * j + c16;
        bj[j] = bias[u];
        rj[j] = RS ? rs[u] : 1.0f;
    }
    float inv[C::TM][4];
#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float amax = 0.f;
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                const float g = gelu_erf(acc[i][j][r] + bj[j]), v = RS ? g * rj[j] : g;
                acc[i][j][r] = v;
                amax = __builtin_fmaxf(amax, __builtin_fabsf(v));
            }
            amax = row16_max(amax);
            const float sc = block_scale(amax);
            inv[i][r] = 1.0f / sc;
            const int m = m0 + wm0 + 16 * i + 4 * g + r;
            if (c16 == 0 && m < rows) ms[(size_t)blk * lds + m] = sc;
        }
    float *tr = (float *)(smem + (threadIdx.x >> 6) * LAYER_RES_SLICE);
    const __amdgpu_buffer_rsrc_t rm = buf_rsrc(m8, (uint32_t)rows * PX_HID);
    const int rsub = lane >> 3, ch = lane & 7;
#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
        if (pass) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the previous pass's slice reads are done
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    tr[(16 * i + 4 * g + r) * 68 + 16 * jj + c16] = acc[i][4 * pass + jj][r] * inv[i][r];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slice is the wave's own: no block barrier needed
#pragma unroll
        for (int it = 0; it < 8; it++) {
            const int rr = 8 * it + rsub;
            const float4 a = *(const float4 *)(tr + rr * 68 + 8 * ch), b = *(const float4 *)(tr + rr * 68 + 8 * ch + 4);
            typedef unsigned v2u __attribute__((ext_vector_type(2)));
            const v2u o = {e4_pack4_scaled(a.x, a.y, a.z, a.w), e4_pack4_scaled(b.x, b.y, b.z, b.w)};
            const uint32_t off = (uint32_t)(m0 + wm0 + rr) * PX_HID + (uint32_t)(128 * blk + 64 * pass + 8 * ch);
            __builtin_amdgcn_raw_buffer_store_b64(o, rm, (int)off, 0, 0);
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// C-ABI launchers
// ---------------------------------------------------------------------------------------------------------------

extern "C" int px_k_qkv(const void *h8, const float *hs, int lds, const void *w, const float *ws, const float *bias,
                        const float *cs, int L, void *q, void *k, void *vt, int rows, void *stream)
{
    if (layer_rows_ok("px_k_qkv", rows, lds)) return -1;
    if (L <= 0 || L % 64 || rows % L) return xt_fail("px_k_qkv", "L must be a positive multiple of 64 dividing rows");
    if (!XT_ALIGNED(h8) || !XT_ALIGNED(w) || ((uintptr_t)bias & 7) || ((uintptr_t)cs & 7))
        return xt_fail("px_k_qkv", "h8 and w must be 16-byte aligned, bias and cs 8-byte aligned");
    hipLaunchKernelGGL(k_px_qkv<false>, dim3(layer_grid(rows, 3 * XT_D, LayerCfg::BM, LayerCfg::BN)),
                       dim3(LayerCfg::NT), 0, (hipStream_t)stream, (const uint8_t *)h8, hs, lds, (const uint8_t *)w,
                       (const uint32_t *)nullptr, ws, bias, cs, L, (uint16_t *)q, (uint16_t *)k, (uint16_t *)vt, rows);
    return xt_check("px_k_qkv");
}

template <int K>
static int px_res_launch(const char *what, const void *a8, const float *as, int lds, const void *w, const float *ws,
                         const float *bias, void *x, int rows, void *stream)
{
    if (layer_rows_ok(what, rows, lds)) return -1;
    if (!XT_ALIGNED(a8) || !XT_ALIGNED(w)) return xt_fail(what, "a8 and w must be 16-byte aligned");
    hipLaunchKernelGGL((k_px_res<false, K>), dim3(layer_grid(rows, XT_D, LayerCfg::BM, LayerCfg::BN)), dim3(LayerCfg::NT),
                       0, (hipStream_t)stream, (const uint8_t *)a8, as, lds, (const uint8_t *)w,
                       (const uint32_t *)nullptr, ws, bias, (uint16_t *)x, rows);
    return xt_check(what);
}

extern "C" int px_k_proj(const void *a8, const float *as, int lds, const void *w, const float *ws, const float *bias,
                         void *x, int rows, void *stream)
{
    return px_res_launch<XT_D>("px_k_proj", a8, as, lds, w, ws, bias, x, rows, stream);
}

extern "C" int px_k_fc2(const void *m8, const float *ms, int lds, const void *w, const float *ws, const float *bias,
                        void *x, int rows, void *stream)
{
    return px_res_launch<PX_HID>("px_k_fc2", m8, ms, lds, w, ws, bias, x, rows, stream);
}

extern "C" int px_k_fc1(const void *h8, const float *hs, int lds, const void *w, const float *ws, const float *bias,
                        const float *rs, void *m8, float *ms, int rows, void *stream)
{
    if (layer_rows_ok("px_k_fc1", rows, lds)) return -1;
    if (!XT_ALIGNED(h8) || !XT_ALIGNED(w) || ((uintptr_t)m8 & 7))
        return xt_fail("px_k_fc1", "h8 and w must be 16-byte aligned, m8 8-byte aligned");
    auto kern = rs ? k_px_fc1<false, true> : k_px_fc1<false, false>;  // the multiply only where rs is given
    hipLaunchKernelGGL(kern, dim3(layer_grid(rows, PX_HID, LayerCfg::BM, LayerCfg::BN)), dim3(LayerCfg::NT), 0,
                       (hipStream_t)stream, (const uint8_t *)h8, hs, lds, (const uint8_t *)w, (const uint32_t *)nullptr,
                       ws, bias, rs, (uint8_t *)m8, ms, rows);
    return xt_check("px_k_fc1");
}

// ---------------------------------------------------------------------------------------------------------------
// Attention-pool head (px_kernels.cu:341-503): the scores s [nb T][16] of k_px_hln -> per (image, head) softmax over
// the T tokens -> pooled = P y -> o = Wv pooled per head; the tag head is then eva_k_quant_act + eva_k_head.
// ---------------------------------------------------------------------------------------------------------------
#define PX_PCH 144  // tokens per pooling chunk (px_kernels.cu:446 PCH)

// k_px_hsoft (k_phsoft, 406-440): P [nb][16][T] fp16 = 2^(s - max) / sum, one block of 256 threads per (image, head);
// the maximum and the sum run per thread in token order, then through the wave butterfly and the 4 waves in order.
__global__ void __launch_bounds__(256) k_px_hsoft(const float *__restrict__ s, uint16_t *__restrict__ P, int T)
{
    __shared__ float red[4];
    const int b = blockIdx.x >> 4, h = blockIdx.x & 15, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const float *sb = s + (size_t)b * T * 16 + h;
    float m = -3.0e38f;
    for (int t = threadIdx.x; t < T; t += 256) m = __builtin_fmaxf(m, sb[(size_t)t * 16]);
    m = wave_max(m);
    if (lane == 0) red[w] = m;
    __syncthreads();
    m = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
    __syncthreads();
    float l = 0.f;
    for (int t = threadIdx.x; t < T; t += 256) l += __builtin_amdgcn_exp2f(sb[(size_t)t * 16] - m);
    l = wave_sum(l);
    if (lane == 0) red[w] = l;
    __syncthreads();
    const float inv = 1.0f / (((red[0] + red[1]) + red[2]) + red[3]);
    for (int t = threadIdx.x; t < T; t += 256)
        P[(size_t)blockIdx.x * T + t] = f2h(__builtin_amdgcn_exp2f(sb[(size_t)t * 16] - m) * inv);
}

// k_px_hpool (k_phpool, 447-473): part [nb][T/144][16][1024] fp32, the sum over one 144-token chunk of P[h][t] y[t][d],
// tokens in order (fma chains); k_px_hv adds the chunks in order. Grid (nb, T/144, 2): 256 threads, two dims each,
// all 16 heads at once, so y is read once; the chunk's P sits in shared memory as [token][head].
__global__ void __launch_bounds__(256) k_px_hpool(const uint16_t *__restrict__ P, const uint16_t *__restrict__ y,
                                                  float *__restrict__ part, int T)
{
    __shared__ __attribute__((aligned(16))) float sp[PX_PCH][16];
    const int b = blockIdx.x, c = blockIdx.y, t0 = c * PX_PCH, d = 512 * blockIdx.z + 2 * threadIdx.x;
    for (int i = threadIdx.x; i < PX_PCH * 16; i += 256) {
        const int h = i / PX_PCH, t = i - h * PX_PCH;
        sp[t][h] = h2f(P[((size_t)b * 16 + h) * T + t0 + t]);
    }
    __syncthreads();
    float a0[16], a1[16];
#pragma unroll
    for (int h = 0; h < 16; h++) a0[h] = a1[h] = 0.f;
    const uint16_t *yr = y + ((size_t)b * T + t0) * XT_D + d;
    for (int t = 0; t < PX_PCH; t++) {
        const uint32_t u = *(const uint32_t *)(yr + (size_t)t * XT_D);
        const float v0 = h2f((uint16_t)(u & 0xffffu)), v1 = h2f((uint16_t)(u >> 16));
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 p = *(const float4 *)&sp[t][4 * q];
            const float pp[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                a0[4 * q + k] = __builtin_fmaf(pp[k], v0, a0[4 * q + k]);
                a1[4 * q + k] = __builtin_fmaf(pp[k], v1, a1[4 * q + k]);
            }
        }
    }
    float *po = part + (((size_t)b * gridDim.y + c) * 16) * XT_D + d;
#pragma unroll
    for (int h = 0; h < 16; h++) *(float2 *)(po + (size_t)h * XT_D) = make_float2(a0[h], a1[h]);
}

// k_px_hv (k_phv, 477-503): pooled[b][h] = the nch chunk partials summed in chunk order, then
// o[b][64 h + n] = f16(Wv[64 h + n] . pooled[b][h]) (Wv fp16 [1024][1024]), written as fp32 holding the fp16 value
// (the reference's fp16 o, ready for eva_k_quant_act). One block of 256 threads per (image, head): each wave takes 16
// outputs, each lane 16 of the 1024 products in element order, met in the butterfly.
__global__ void __launch_bounds__(256) k_px_hv(const float *__restrict__ part, int nch, const uint16_t *__restrict__ wv,
                                               float *__restrict__ o)
{
    __shared__ __attribute__((aligned(16))) float pv[XT_D];
    const int b = blockIdx.x >> 4, h = blockIdx.x & 15, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    {
        const float *pp = part + ((size_t)b * nch * 16 + h) * XT_D + 4 * threadIdx.x;
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int c = 0; c < nch; c++) {
            const float4 v = *(const float4 *)(pp + (size_t)c * 16 * XT_D);
            a.x += v.x;
            a.y += v.y;
            a.z += v.z;
            a.w += v.w;
        }
        *(float4 *)(pv + 4 * threadIdx.x) = a;
    }
    __syncthreads();
    float x[16];
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        const float4 a = *(const float4 *)(pv + 512 * hh + 8 * lane), c = *(const float4 *)(pv + 512 * hh + 8 * lane + 4);
        x[8 * hh + 0] = a.x; x[8 * hh + 1] = a.y; x[8 * hh + 2] = a.z; x[8 * hh + 3] = a.w;
        x[8 * hh + 4] = c.x; x[8 * hh + 5] = c.y; x[8 * hh + 6] = c.z; x[8 * hh + 7] = c.w;
    }
    float mine = 0.f;
    for (int k = 0; k < 16; k++) {
        const int n = 64 * h + 16 * w + k;
        float a = 0.f;
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const uint4 u = *(const uint4 *)(wv + (size_t)n * XT_D + 512 * hh + 8 * lane);
            const uint32_t ww[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                a = __builtin_fmaf(h2f((uint16_t)(ww[i] & 0xffffu)), x[8 * hh + 2 * i], a);
                a = __builtin_fmaf(h2f((uint16_t)(ww[i] >> 16)), x[8 * hh + 2 * i + 1], a);
            }
        }
        a = wave_sum(a);
        mine = lane == k ? a : mine;
    }
    if (lane < 16) o[(size_t)b * XT_D + 64 * h + 16 * w + lane] = h2f(f2h(mine));
}

extern "C" int px_k_hsoft(const float *s, void *P, int nb, int T, void *stream)
{
    if (nb <= 0 || T <= 0) return xt_fail("px_k_hsoft", "bad shape (nb > 0, T > 0)");
    hipLaunchKernelGGL(k_px_hsoft, dim3(nb * 16), dim3(256), 0, (hipStream_t)stream, s, (uint16_t *)P, T);
    return xt_check("px_k_hsoft");
}

extern "C" int px_k_hpool(const void *P, const void *y, float *part, int nb, int T, void *stream)
{
    if (nb <= 0 || T <= 0 || T % PX_PCH) return xt_fail("px_k_hpool", "T must be a positive multiple of 144");
    if (((uintptr_t)y & 3) || ((uintptr_t)part & 7)) return xt_fail("px_k_hpool", "y 4-byte, part 8-byte aligned");
    hipLaunchKernelGGL(k_px_hpool, dim3(nb, T / PX_PCH, 2), dim3(256), 0, (hipStream_t)stream, (const uint16_t *)P,
                       (const uint16_t *)y, part, T);
    return xt_check("px_k_hpool");
}

extern "C" int px_k_hv(const float *part, int nch, const void *wv, float *o, int nb, void *stream)
{
    if (nb <= 0 || nch <= 0) return xt_fail("px_k_hv", "bad shape (nb > 0, nch > 0)");
    if (((uintptr_t)part | (uintptr_t)wv) & 15) return xt_fail("px_k_hv", "part and wv must be 16-byte aligned");
    hipLaunchKernelGGL(k_px_hv, dim3(nb * 16), dim3(256), 0, (hipStream_t)stream, part, nch, (const uint16_t *)wv, o);
    return xt_check("px_k_hv");
}

// GELU of n fp32 values by the fc1 epilogue's gelu_erf (test hook: its accuracy is not visible through the E4M3 output)
__global__ void __launch_bounds__(256) k_px_gelu(const float *__restrict__ u, float *__restrict__ g, int n)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) g[i] = gelu_erf(u[i]);
}

extern "C" int px_probe_gelu(const float *u, float *g, int n, void *stream)
{
    if (n <= 0) return xt_fail("px_probe_gelu", "n must be positive");
    hipLaunchKernelGGL(k_px_gelu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, u, g, n);
    return xt_check("px_probe_gelu");
}
