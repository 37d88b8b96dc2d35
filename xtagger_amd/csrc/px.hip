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
// free: with t = |u|, Phi(-t) = 2^Q(t), Q(t) = -t^2 / (2 ln 2) + R(s), R a degree-7 polynomial in s = min(t / 6, 1),
// the minimax fit (Remez exchange) to log2 Phi(-t) + t^2 / (2 ln 2) on [0, 6] (|R error| 4.7e-6); then
// u Phi(u) = max(u, 0) - t Phi(-t) (u Phi(-t) for u < 0, u (1 - Phi(-t)) otherwise: Phi(u) + Phi(-u) = 1), one fma
// with no cancellation on either side. In fp32 against float64: Phi(-t) within 5.2e-6 relative on [0, 6] (R's error
// and the rounding of Q), so u Phi(u) within 3.4e-6 relative for u >= 0. Past t = 6 R is held at R(6): Phi(-t) < 1e-9
// there and comes out too large by at most a factor t / 6. s is one multiply with the output clamp; the whole GELU is
// one v_exp_f32 and 12 other instructions, where erff takes two divergent branches.
__device__ __forceinline__ float gelu_erf(float u)
{
    const float t = __builtin_fabsf(u), s = __builtin_fminf(__builtin_fmaxf(t * 0.166666672f, 0.0f), 1.0f);
    float r = -5.136296153e-01f;
    r = __builtin_fmaf(r, s, 2.873929501e+00f);
    r = __builtin_fmaf(r, s, -7.235760689e+00f);
    r = __builtin_fmaf(r, s, 1.102622604e+01f);
    r = __builtin_fmaf(r, s, -1.165537453e+01f);
    r = __builtin_fmaf(r, s, 9.463792801e+00f);
    r = __builtin_fmaf(r, s, -6.907506466e+00f);
    r = __builtin_fmaf(r, s, -9.999952912e-01f);
    const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(-0.72134752f, t * t, r));  // Phi(-t)
    return __builtin_fmaf(-t, e, __builtin_fmaxf(u, 0.0f));
}

// ---------------------------------------------------------------------------------------------------------------
// k_px_qkv: h8 [rows][1024] x Wqkv [3072][1024] + bias -> q, k bf16 [S][16][L][64] (RoPE on every token with table
// row t = m % L, cs [L][32] (cos, sin) of pair i = dims 2i, 2i+1), vt bf16 [S][16][64][L]; rows = S L. Weight rows of
// q and k are quad-split as for the wd model (column tile j of a head holds dim 4i + j, i = lane & 15: a lane holds
// pairs 2i and 2i + 1 whole); the bias stays in natural order. q rows of W and of the bias carry log2(e)/8 (the
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
        v4f bq[2];  // bias of dims 4 c16 .. 4 c16 + 3 of each head
#pragma unroll
        for (int hh = 0; hh < 2; hh++) bq[hh] = *(const v4f *)(bias + part * XT_D + (head0 + hh) * XT_HD + 4 * c16);
        v4f rot[C::TM][4];  // (cos, sin) of pairs 2 c16 and 2 c16 + 1
        uint32_t base[C::TM][4];  // element offset of (sequence, head head0, token), dims 0
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm0 + 16 * i + 4 * g + r, s = m / L, t = m - s * L;
                base[i][r] = ((uint32_t)(s * XT_NH + head0) * (uint32_t)L + (uint32_t)t) * XT_HD;
                rot[i][r] = __builtin_bit_cast(
                    v4f, __builtin_amdgcn_raw_buffer_load_b128(rc, (int)(((uint32_t)t * 32u + 2 * c16) * 8u), 0, 0));
            }
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    uint32_t two[2];
#pragma unroll
                    for (int p = 0; p < 2; p++) {
                        const float f0 = acc[i][4 * hh + 2 * p][r] + bq[hh][2 * p];
                        const float f1 = acc[i][4 * hh + 2 * p + 1][r] + bq[hh][2 * p + 1];
                        const float cr = rot[i][r][2 * p], sr = rot[i][r][2 * p + 1];
                        const float g0 = __builtin_fmaf(f0, cr, -(f1 * sr)), g1 = __builtin_fmaf(f1, cr, f0 * sr);
                        two[p] = pk_bf16(g0, g1);
                    }
                    const uint32_t off = (base[i][r] + (uint32_t)(hh * L * XT_HD + 4 * c16)) * 2u;
                    typedef unsigned v2u __attribute__((ext_vector_type(2)));
                    __builtin_amdgcn_raw_buffer_store_b64(v2u{two[0], two[1]}, rd, (int)off, 0, 0);
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
    // the tile transposed (TR): lane (g, c16) holds columns n0 + wn0 + 16 j + 4 g + r, one 16-byte bias load per j
    layer_mainloop<C, SP, BsNoPre, true>(a8, K, as, lds, w, wx, ws, rows, XT_D, K, m0, n0, smem, acc);
    bs_wave_origin<C>(wm0, wn0);
    const int g = (threadIdx.x & 63) >> 4;
    float4 b4[C::TN];
#pragma unroll
    for (int j = 0; j < C::TN; j++) b4[j] = *(const float4 *)(bias + n0 + wn0 + 16 * j + 4 * g);
    residual_add_t<C>(smem, [&](int j, int i) {
        const v4f v = acc[i][j];
        return v4f{v[0] + b4[j].x, v[1] + b4[j].y, v[2] + b4[j].z, v[3] + b4[j].w};
    }, x, m0 + wm0, n0 + wn0, rows);
}

// ---------------------------------------------------------------------------------------------------------------
// k_px_fc1: h8 [rows][1024] x W1 [4736][1024] -> h = rs (gelu(acc + b1)), gelu(u) = u Phi(u) (exact normal CDF,
// px_kernels.cu:228-231, by gelu_erf; rs may be NULL = 1), packed to m8 [rows][4736] E4M3 with 1x128 scales
// ms [37][lds]. A wave's 128 columns are one scale block: each row's |max| meets in a 4-lane reduction (the tile is
// transposed), the values are scaled in registers, parked in the wave's own LDS slice 64 columns at a time and stored 8 consecutive
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
    // the tile transposed (TR): lane (g, c16) holds row m0 + wm0 + 16 i + c16 and units 128 blk + 16 j + 4 g + r, so
    // a row's 128 units lie in the 4 lanes that share c16: its |max| meets in two lane swaps, one scale per lane and
    // row tile
    layer_mainloop<C, SP, BsNoPre, true>(h8, XT_D, hs, lds, w, wx, ws, rows, PX_HID, XT_D, m0, n0, smem, acc);
    bs_wave_origin<C>(wm0, wn0);
    const int blk = (n0 + wn0) >> 7;
    if (blk >= PX_HID / 128) return;  // no block barrier follows: the epilogue uses the wave's own slice only
    const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    float4 b4[C::TN], r4[C::TN];
#pragma unroll
    for (int j = 0; j < C::TN; j++) {
        const int u = 128 * blk + 16 * j + 4 * g;
        b4[j] = *(const float4 *)(bias + u);
        r4[j] = RS ? *(const float4 *)(rs + u) : make_float4(1.f, 1.f, 1.f, 1.f);
    }
    float inv[C::TM];
#pragma unroll
    for (int i = 0; i < C::TM; i++) {
        float amax = 0.f;
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
            const float bb[4] = {b4[j].x, b4[j].y, b4[j].z, b4[j].w}, rr[4] = {r4[j].x, r4[j].y, r4[j].z, r4[j].w};
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float g = gelu_erf(acc[i][j][r] + bb[r]), v = RS ? g * rr[r] : g;
                acc[i][j][r] = v;
                amax = __builtin_fmaxf(amax, __builtin_fabsf(v));
            }
        }
        amax = col4_absmax(amax);
        const float sc = block_scale(amax);
        inv[i] = block_scale_inv(sc);
        const int m = m0 + wm0 + 16 * i + c16;
        if (g == 0 && m < rows) ms[(size_t)blk * lds + m] = sc;
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
            for (int jj = 0; jj < 4; jj++) {
                const v4f v = acc[i][4 * pass + jj];
                *(float4 *)(tr + (16 * i + c16) * 68 + 16 * jj + 4 * g) =
                    make_float4(v[0] * inv[i], v[1] * inv[i], v[2] * inv[i], v[3] * inv[i]);
            }
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
// Attention-pool head (px_kernels.cu:341-503, px.h:170-189): the scores s [nb T][16] of k_px_hln (exp2 domain) ->
// per (image, head) softmax weights over the T tokens, rounded to fp16 as the reference's P -> pooled = P y per head
// -> o = Wv pooled per head. Three launches, each over the whole batch:
//   k_px_hstat  (image, 576-token window): each head's maximum over the window and sum of 2^(s - maximum)
//   k_px_hpool  (image, 288-token window, 128 columns of y) per wave: P made in registers from s and the merged
//               statistics; P y on v_mfma_f32_16x16x32_f16, the 16 heads being the MFMA's 16 rows, eight 16 x 16
//               output tiles per wave -> an fp32 partial per window
//   k_px_hproj  (head, 2 images): the window partials summed in window order, then the head's value projection,
//               fp16 result
// Every sum runs in an order fixed by the launch shape, so results repeat bit for bit. The tag head follows as
// eva_k_quant_act + eva_k_head.
// ---------------------------------------------------------------------------------------------------------------
constexpr int PX_PW = 576;  // tokens per statistics window

// stat [nb][T / 576][16] float2 = (m, l): m = the window's maximum of s[.][h], l = sum_t 2^(s[t][h] - m). Thread
// 4 r + q holds heads 4q .. 4q + 3 of tokens r, r + 64, .., r + 512 in registers (one read of the window); its nine
// terms are added in token order, then across the 16 lanes of the same q by the xor butterfly, then waves 0 .. 3.
__global__ void __launch_bounds__(256) k_px_hstat(const float *__restrict__ s, float2 *__restrict__ stat, int T)
{
    __shared__ float rm[4][16], rl[4][16];
    const int w = blockIdx.x, b = blockIdx.y, q = threadIdx.x & 3, r = threadIdx.x >> 2;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const float4 *sw = (const float4 *)(s + ((size_t)b * T + (size_t)w * PX_PW) * 16);
    float v[PX_PW / 64][4];
#pragma unroll
    for (int i = 0; i < PX_PW / 64; i++) {
        const float4 a = sw[(size_t)(r + 64 * i) * 4 + q];
        v[i][0] = a.x, v[i][1] = a.y, v[i][2] = a.z, v[i][3] = a.w;
    }
    float m[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        m[e] = v[0][e];
#pragma unroll
        for (int i = 1; i < PX_PW / 64; i++) m[e] = __builtin_fmaxf(m[e], v[i][e]);
#pragma unroll
        for (int o = 4; o < 64; o <<= 1) m[e] = __builtin_fmaxf(m[e], __shfl_xor(m[e], o));
    }
    if (lane < 4)
#pragma unroll
        for (int e = 0; e < 4; e++) rm[wv][4 * q + e] = m[e];
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int h = 4 * q + e;
        m[e] = __builtin_fmaxf(__builtin_fmaxf(rm[0][h], rm[1][h]), __builtin_fmaxf(rm[2][h], rm[3][h]));
        l[e] = 0.f;
#pragma unroll
        for (int i = 0; i < PX_PW / 64; i++) l[e] += __builtin_amdgcn_exp2f(v[i][e] - m[e]);
#pragma unroll
        for (int o = 4; o < 64; o <<= 1) l[e] += __shfl_xor(l[e], o);
    }
    if (lane < 4)
#pragma unroll
        for (int e = 0; e < 4; e++) rl[wv][4 * q + e] = l[e];
    __syncthreads();
    if (threadIdx.x < 16) {
        const int h = threadIdx.x;
        stat[((size_t)b * gridDim.x + w) * 16 + h] =
            make_float2(__builtin_fmaxf(__builtin_fmaxf(rm[0][h], rm[1][h]), __builtin_fmaxf(rm[2][h], rm[3][h])),
                        (rl[0][h] + rl[1][h]) + (rl[2][h] + rl[3][h]));
    }
}

// part [nb][T / 288][16][1024] fp32 = sum over pooling window w (288 tokens) of P[h][t] y[t][d], one wave per
// (image, window, 128 columns), no shared memory. Head h's statistics merge in window order: M = max_i m_i,
// L = sum_i l_i 2^(m_i - M) (every lane of head h, the 576-token windows read through a buffer resource that ends at
// the image's last one). Lane (g, c), head h = c:
//   A fragment of K step k = P[h][32 k + 8 g + e], e < 8: f16(2^(s - M) / L) of the lane's own eight scores;
//   B fragments: the lane loads y[32 k + 8 g + e][col0 + 8 c .. + 7] (16 bytes, a 256-byte row segment per 16 lanes)
//   for its eight tokens and transposes the 8 x 8 halves in registers (v_perm_b32), so tile q in 0 .. 7 holds columns
//   col0 + 8 c + q and one y load feeds one MFMA; three K steps of scores and y are in flight ahead of the MFMAs.
// P (optional, fp16 [nb][16][T]) is written by the waves of the first column group.
constexpr int PX_QW = 288;     // tokens per pooling window
constexpr int PX_PWMAX = 16;   // statistics windows per image (T <= 9216)
__global__ void __launch_bounds__(256) k_px_hpool(const float *__restrict__ s, const float2 *__restrict__ stat,
                                                  const uint16_t *__restrict__ y, uint16_t *__restrict__ P,
                                                  float *__restrict__ part, int T)
{
    constexpr int KS = PX_QW / 32, DEPTH = 3;
    const int w = blockIdx.y, b = blockIdx.z, nq = gridDim.y, nw = T / PX_PW, lane = threadIdx.x & 63;
    const int g = lane >> 4, c = lane & 15, col0 = 512 * blockIdx.x + 128 * (threadIdx.x >> 6);
    const size_t tok0 = (size_t)b * T + (size_t)w * PX_QW;
    const __amdgpu_buffer_rsrc_t rst = buf_rsrc(stat + (size_t)b * nw * 16, (uint32_t)nw * 16 * 8);
    v2f sv[PX_PWMAX];
#pragma unroll
    for (int i = 0; i < PX_PWMAX; i++)
        sv[i] = __builtin_bit_cast(v2f, __builtin_amdgcn_raw_buffer_load_b64(rst, (16 * i + c) * 8, 0, 0));
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(s + tok0 * 16, PX_QW * 16 * 4);
    const __amdgpu_buffer_rsrc_t ry = buf_rsrc(y + tok0 * XT_D, PX_QW * XT_D * 2);
    const int soff = (8 * g * 16 + c) * 4, yoff = (8 * g * XT_D + col0 + 8 * c) * 2;
    float sk[KS][8];
    uint4 yk[KS][8];
#pragma unroll
    for (int k = 0; k < DEPTH; k++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            sk[k][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, soff, (32 * k + e) * 64, 0));
            yk[k][e] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ry, yoff, (32 * k + e) * XT_D * 2, 0));
        }
    float mx = sv[0][0], l = 0.f;
#pragma unroll
    for (int i = 1; i < PX_PWMAX; i++) mx = i < nw ? __builtin_fmaxf(mx, sv[i][0]) : mx;
#pragma unroll
    for (int i = 0; i < PX_PWMAX; i++) l = i < nw ? l + sv[i][1] * __builtin_amdgcn_exp2f(sv[i][0] - mx) : l;
    const float inv = 1.0f / l;
    v4f acc[8];
#pragma unroll
    for (int q = 0; q < 8; q++) acc[q] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < KS; k++) {
        uint32_t pa[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
            pa[i] = (uint32_t)f2h(__builtin_amdgcn_exp2f(sk[k][2 * i] - mx) * inv) |
                    ((uint32_t)f2h(__builtin_amdgcn_exp2f(sk[k][2 * i + 1] - mx) * inv) << 16);
        const v8h a = __builtin_bit_cast(v8h, make_uint4(pa[0], pa[1], pa[2], pa[3]));
        if (P && col0 == 0)
            *(uint4 *)(P + ((size_t)b * 16 + c) * T + (size_t)w * PX_QW + 32 * k + 8 * g) = make_uint4(pa[0], pa[1], pa[2], pa[3]);
#pragma unroll
        for (int m = 0; m < 4; m++) {  // columns 2m (low halves) and 2m + 1 (high halves) of the eight tokens
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t r0 = ((const uint32_t *)&yk[k][2 * i])[m], r1 = ((const uint32_t *)&yk[k][2 * i + 1])[m];
                lo[i] = __builtin_amdgcn_perm(r1, r0, 0x05040100u);
                hi[i] = __builtin_amdgcn_perm(r1, r0, 0x07060302u);
            }
            acc[2 * m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(v8h, make_uint4(lo[0], lo[1], lo[2], lo[3])), acc[2 * m], 0, 0, 0);
            acc[2 * m + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(v8h, make_uint4(hi[0], hi[1], hi[2], hi[3])), acc[2 * m + 1], 0, 0, 0);
        }
        if (k + DEPTH < KS)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                sk[k + DEPTH][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, soff, (32 * (k + DEPTH) + e) * 64, 0));
                yk[k + DEPTH][e] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ry, yoff, (32 * (k + DEPTH) + e) * XT_D * 2, 0));
            }
    }
    // acc[q][r] = head 4 g + r, column col0 + 8 c + q
    float *po = part + (((size_t)b * nq + w) * 16 + 4 * g) * XT_D + col0 + 8 * c;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        *(float4 *)(po + (size_t)r * XT_D) = make_float4(acc[0][r], acc[1][r], acc[2][r], acc[3][r]);
        *(float4 *)(po + (size_t)r * XT_D + 4) = make_float4(acc[4][r], acc[5][r], acc[6][r], acc[7][r]);
    }
}

// o [nb][1024] = f16(Wv[64 h + n] . pooled[b][h]) held as fp32 (ready for eva_k_quant_act), pooled[b][h] = the nw
// window partials summed in window order. Block (head h, images 2 z, 2 z + 1), 256 threads. Thread (image t >> 7,
// columns 8 (t & 127) ..) reads its partials four windows at a time through a buffer resource that ends at the image's
// last window, so reads past it return zeros and every load of a round is in flight at once; the two pooled rows sit in
// shared memory as [image][half][512 + 4]. Then thread (n, image, half) = (t >> 2, (t >> 1) & 1, t & 1) takes row
// 64 h + n of Wv over its half of the columns as two interleaved fma chains, and one xor shuffle adds the halves.
__global__ void __launch_bounds__(256) k_px_hproj(const float *__restrict__ part, int nw, const uint16_t *__restrict__ wv,
                                                  float *__restrict__ o, int nb)
{
    constexpr int HS = XT_D / 2 + 4;
    __shared__ __attribute__((aligned(16))) float pl[2 * 2 * HS];
    const int h = blockIdx.x, b0 = 2 * blockIdx.y, t = threadIdx.x;
    {
        const int bi = __builtin_amdgcn_readfirstlane(t >> 7), d = 8 * (t & 127);  // bi is the same in a wave
        const bool live = b0 + bi < nb;
        const __amdgpu_buffer_rsrc_t rp = buf_rsrc(part + (size_t)(live ? b0 + bi : 0) * nw * 16 * XT_D,
                                                   live ? (uint32_t)nw * 16 * XT_D * 4 : 0u);
        float4 a0 = make_float4(0.f, 0.f, 0.f, 0.f), a1 = a0;
        for (int i0 = 0; i0 < nw; i0 += 4) {
            float4 v0[4], v1[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int off = (((i0 + k) * 16 + h) * XT_D + d) * 4;
                v0[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rp, off, 0, 0));
                v1[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rp, off + 16, 0, 0));
            }
#pragma unroll
            for (int k = 0; k < 4; k++) {
                a0.x += v0[k].x, a0.y += v0[k].y, a0.z += v0[k].z, a0.w += v0[k].w;
                a1.x += v1[k].x, a1.y += v1[k].y, a1.z += v1[k].z, a1.w += v1[k].w;
            }
        }
        float *dst = pl + (2 * bi + d / (XT_D / 2)) * HS + d % (XT_D / 2);
        *(float4 *)dst = a0;
        *(float4 *)(dst + 4) = a1;
    }
    __syncthreads();
    const int n = t >> 2, bi = (t >> 1) & 1, half = t & 1;
    const uint16_t *wr = wv + (size_t)(64 * h + n) * XT_D + (XT_D / 2) * half;
    const float *pr = pl + (2 * bi + half) * HS;
    float a0 = 0.f, a1 = 0.f;
#pragma unroll 4
    for (int k = 0; k < XT_D / 2; k += 16) {
        const uint4 u0 = *(const uint4 *)(wr + k), u1 = *(const uint4 *)(wr + k + 8);
        const uint32_t w0[4] = {u0.x, u0.y, u0.z, u0.w}, w1[4] = {u1.x, u1.y, u1.z, u1.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float2 p0 = *(const float2 *)(pr + k + 2 * i), p1 = *(const float2 *)(pr + k + 8 + 2 * i);
            a0 = __builtin_fmaf(h2f((uint16_t)(w0[i] & 0xffffu)), p0.x, a0);
            a0 = __builtin_fmaf(h2f((uint16_t)(w0[i] >> 16)), p0.y, a0);
            a1 = __builtin_fmaf(h2f((uint16_t)(w1[i] & 0xffffu)), p1.x, a1);
            a1 = __builtin_fmaf(h2f((uint16_t)(w1[i] >> 16)), p1.y, a1);
        }
    }
    float a = a0 + a1;
    a += __shfl_xor(a, 1);
    if (!half && b0 + bi < nb) o[(size_t)(b0 + bi) * XT_D + 64 * h + n] = h2f(f2h(a));
}

extern "C" int px_k_hstat(const float *s, float *stat, int nb, int T, void *stream)
{
    if (nb <= 0 || T <= 0 || T % PX_PW || T / PX_PW > 65535 || nb > 65535)
        return xt_fail("px_k_hstat", "T must be a positive multiple of 576, nb in 1 .. 65535");
    if (((uintptr_t)s & 15) || ((uintptr_t)stat & 7)) return xt_fail("px_k_hstat", "s 16-byte, stat 8-byte aligned");
    hipLaunchKernelGGL(k_px_hstat, dim3(T / PX_PW, nb), dim3(256), 0, (hipStream_t)stream, s, (float2 *)stat, T);
    return xt_check("px_k_hstat");
}

extern "C" int px_k_hpool(const float *s, const float *stat, const void *y, void *P, float *part, int nb, int T,
                          void *stream)
{
    if (nb <= 0 || T <= 0 || T % PX_PW || T / PX_PW > PX_PWMAX || nb > 65535)
        return xt_fail("px_k_hpool", "T must be a positive multiple of 576 up to 9216, nb in 1 .. 65535");
    if (((uintptr_t)s | (uintptr_t)P | (uintptr_t)y | (uintptr_t)part) & 15 || ((uintptr_t)stat & 7))
        return xt_fail("px_k_hpool", "s, P, y and part must be 16-byte aligned, stat 8-byte");
    hipLaunchKernelGGL(k_px_hpool, dim3(XT_D / 512, T / PX_QW, nb), dim3(256), 0, (hipStream_t)stream, s,
                       (const float2 *)stat, (const uint16_t *)y, (uint16_t *)P, part, T);
    return xt_check("px_k_hpool");
}

extern "C" int px_k_hproj(const float *part, int nw, const void *wv, float *o, int nb, void *stream)
{
    if (nb <= 0 || nw <= 0 || nw > 2 * PX_PWMAX || nb > 2 * 65535)
        return xt_fail("px_k_hproj", "bad shape (nb > 0, 0 < nw <= 32)");
    if (((uintptr_t)part | (uintptr_t)wv) & 15) return xt_fail("px_k_hproj", "part and wv must be 16-byte aligned");
    hipLaunchKernelGGL(k_px_hproj, dim3(16, (nb + 1) / 2), dim3(256), 0, (hipStream_t)stream, part, nw,
                       (const uint16_t *)wv, o, nb);
    return xt_check("px_k_hproj");
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
