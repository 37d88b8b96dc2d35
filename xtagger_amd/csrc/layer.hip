// layer.hip - the EVA02-L block GEMMs with their fused epilogues, all on the block-scaled main loop (gemm_core.h),
// plus the fp16 patch embedding. Reference roles (src/engine/eva_kernels.cu): k_qkv (41-114), k_oproj (134-162),
// k_fc1 (211-279), k_fc2 (286-334), k_pe + k_embed (126-130, 21-33), and the head k_headmv
// (src/engine/kern_common.cuh:679-727) as a block-scaled FP8 GEMM.
//
// Token rows: m = 1025 b + t for image b, token t (t = 0 is cls). Activations E4M3 [rows][K] with 1x128 scale
// planes [K/128][lds]; residual x fp16 [rows][1024].
#include "layer_core.h"


// ---------------------------------------------------------------------------------------------------------------
// k_qkv: h8 [rows][1024] x Wqkv [3072][1024] -> q, k bf16 [nb][16][1088][64] (RoPE on patch tokens), vt bf16
// [nb][16][64][1088]. A 256-column block is 4 heads of one of q | k | v; each wave owns two heads. The weight rows
// of q and k heads are stored quad-split (eva_k_prep_w perm 1): within a head, column tile j holds dim 4i + j for
// i = lane & 15, so a lane holds dims 4i .. 4i + 3, the rotary pairs 2i and 2i + 1 whole: their (cos, sin) come in one
// 16-byte load and the rotated dims leave in one 8-byte store. q rows carry log2(e)/8 (export_eva.py:71).
// ---------------------------------------------------------------------------------------------------------------
template <bool SP>
__global__ void __launch_bounds__(LayerCfg::NT) k_qkv(const uint8_t *__restrict__ h8, const float *__restrict__ hs,
                                                     int lds, const uint8_t *__restrict__ w,
                                                     const uint32_t *__restrict__ wx,
                                                     const float *__restrict__ ws, const float *__restrict__ cs,
                                                     uint16_t *__restrict__ q, uint16_t *__restrict__ k,
                                                     uint16_t *__restrict__ vt, int rows)
{
    using C = LayerCfg;
    __shared__ __attribute__((aligned(16))) uint8_t smem[LAYER_SMEM];
    v4f acc[C::TM][C::TN];
    int m0, n0, wm0, wn0;
    layer_tile<C>(rows, 3 * XT_D, m0, n0);
    args_resident(cs, q, k, vt, lds, rows);
    bs_wave_origin<C>(wm0, wn0);
    const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    const int part = n0 >> 10, head0 = ((n0 & 1023) + wn0) >> 6;
    // v: the wave's 64 rows x 128 dims (two heads) are transposed through its own LDS slice ([128 dims][68] bf16,
    // padded rows), then lanes walk rows (consecutive tokens). The slice takes the tile in whichever layout the main
    // loop leaves it: the sparse loop's transposed tile directly (no pass through the dense layout first), the dense
    // tile as one 8-byte write of four consecutive tokens per (row tile, column tile).
    uint16_t *tr = (uint16_t *)(smem + (threadIdx.x >> 6) * 128 * 68 * 2);
    auto v_out = [&]() {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const int m = m0 + wm0 + lane;
        if (m < rows) {
            const int b = m / XT_T, t = m - b * XT_T;
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                uint16_t *dst = vt + ((size_t)b * XT_NH + head0 + hh) * XT_HD * XT_TP + t;
#pragma unroll 8
                for (int d = 0; d < XT_HD; d++) dst[(size_t)d * XT_TP] = tr[(64 * hh + d) * 68 + lane];
            }
        }
    };
    if constexpr (SP) {
        if (part == 2) {  // a separate copy of the sparse loop: its transposed tile goes straight into the slice
            v4f accT[C::TN][C::TM];  // accT[j][i][r]: dim 16 j + 4 g + r, row 16 i + c16 of the wave tile
            bs_mainloop_sp_t<C>(h8, XT_D, hs, lds, w, wx, ws, rows, 3 * XT_D, XT_D, m0, n0, smem, accT);
#pragma unroll
            for (int j = 0; j < C::TN; j++)
#pragma unroll
                for (int i = 0; i < C::TM; i++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        tr[(16 * j + 4 * g + r) * 68 + 16 * i + c16] = (uint16_t)pk_bf16(accT[j][i][r], 0.f);
            v_out();
            return;
        }
    }
    layer_mainloop<C, SP>(h8, XT_D, hs, lds, w, wx, ws, rows, 3 * XT_D, XT_D, m0, n0, smem, acc);
    if (part < 2) {
        // every (cos, sin) pair of the tile is loaded before the first store: one memory round trip. Patch token t of
        // image b uses row t - 1 of the table (eva_kernels.cu:74-79); cls rows (t = 0) load an out-of-range offset
        // (zero) and are not rotated. Stores go through a descriptor that ends at image nb: rows past `rows` are
        // dropped without a branch.
        const int nbi = rows / XT_T;
        const __amdgpu_buffer_rsrc_t rc = buf_rsrc(cs, 1024u * 32u * 8u);
        const __amdgpu_buffer_rsrc_t rd = buf_rsrc(part ? k : q, (uint32_t)nbi * XT_NH * XT_TP * XT_HD * 2u);
        v4f rot[C::TM][4];  // (cos, sin) of pairs 2 c16 and 2 c16 + 1
        int tok[C::TM][4], img[C::TM][4];
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm0 + 16 * i + 4 * g + r, b = m / XT_T, t = m - b * XT_T;
                img[i][r] = b;
                tok[i][r] = t;
                rot[i][r] = __builtin_bit_cast(
                    v4f, __builtin_amdgcn_raw_buffer_load_b128(rc, (int)(((uint32_t)(t - 1) * 32u + 2 * c16) * 8u), 0, 0));
            }
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int b = img[i][r], t = tok[i][r];
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    uint32_t two[2];
#pragma unroll
                    for (int p = 0; p < 2; p++) {
                        float f0 = acc[i][4 * hh + 2 * p][r], f1 = acc[i][4 * hh + 2 * p + 1][r];
                        if (t) {  // one rounded product and one fma per rotated value
                            const float cr = rot[i][r][2 * p], sr = rot[i][r][2 * p + 1];
                            const float g0 = __builtin_fmaf(f0, cr, -(f1 * sr));
                            f1 = __builtin_fmaf(f1, cr, f0 * sr);
                            f0 = g0;
                        }
                        two[p] = pk_bf16(f0, f1);
                    }
                    const uint32_t off = (uint32_t)((((size_t)b * XT_NH + head0 + hh) * XT_TP + t) * XT_HD + 4 * c16) * 2u;
                    typedef unsigned v2u __attribute__((ext_vector_type(2)));
                    __builtin_amdgcn_raw_buffer_store_b64(v2u{two[0], two[1]}, rd, (int)off, 0, 0);
                }
            }
        return;
    }
    // v (dense tile): rows 16 i + 4 g + r of dim 16 j + c16 are four consecutive tokens of one slice row
#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
            typedef unsigned v2u __attribute__((ext_vector_type(2)));
            *(v2u *)(tr + (16 * j + c16) * 68 + 16 * i + 4 * g) =
                v2u{pk_bf16(acc[i][j][0], acc[i][j][1]), pk_bf16(acc[i][j][2], acc[i][j][3])};
        }
    v_out();
}

// ---------------------------------------------------------------------------------------------------------------
// k_oproj: x [rows][1024] = f16(x + attn_out . Wo^T) (eva_kernels.cu:150-160, alpha folded into the block scales)
// ---------------------------------------------------------------------------------------------------------------
template <bool SP>
__global__ void __launch_bounds__(LayerCfg::NT) k_oproj(const uint8_t *__restrict__ a8, const float *__restrict__ as,
                                                       int lds, const uint8_t *__restrict__ w,
                                                       const uint32_t *__restrict__ wx,
                                                       const float *__restrict__ ws, uint16_t *__restrict__ x, int rows)
{
    using C = LayerCfg;
    __shared__ __attribute__((aligned(16))) uint8_t smem[LAYER_SMEM];
    v4f acc[C::TM][C::TN];
    int m0, n0, wm0, wn0;
    layer_tile<C>(rows, XT_D, m0, n0);
    args_resident(x, lds, rows);
    // the transposed tile (sparse: as the sparse main loop leaves it; dense: TR) goes straight into the residual update
    if constexpr (SP) {
        static_assert(C::LDS_SP <= LAYER_ROWSTAT, "sparse stages end before the row statistics");
        v4f accT[C::TN][C::TM];
        bs_mainloop_sp_t<C>(a8, XT_D, as, lds, w, wx, ws, rows, XT_D, XT_D, m0, n0, smem, accT);
        bs_wave_origin<C>(wm0, wn0);
        residual_add_t<C>(smem, [&](int jn, int im) { return accT[jn][im]; }, x, m0 + wm0, n0 + wn0, rows);
    } else {
        layer_mainloop<C, SP, BsNoPre, true>(a8, XT_D, as, lds, w, wx, ws, rows, XT_D, XT_D, m0, n0, smem, acc);
        bs_wave_origin<C>(wm0, wn0);
        residual_add_t<C>(smem, [&](int jn, int im) { return acc[im][jn]; }, x, m0 + wm0, n0 + wn0, rows);
    }
}

// ---------------------------------------------------------------------------------------------------------------
// k_fc1: h8 [rows][1024] x W12 [5632][1024] -> SwiGLU h = silu(g) x (silu(g) = g / (1 + e^-g), the quotient by the
// hardware reciprocal, within 1 ulp), packed to
// m8 [rows][2816] E4M3 with 1x128 scales ms [22][lds], and per-(row, block) (sum h, sum h^2) of the unpacked h in
// stat [22][lds][2] for the folded MLP LayerNorm (eva_kernels.cu:211-279). W12 rows hold g and x of 16 units in
// alternate 16-row chunks (export_eva.py:60-62), so column tile 2c is g and 2c+1 is x of the same 16 units: a
// 256-column block is one 128-unit block of h; its rows are staged in LDS, where 8 threads per row take the |max|
// and the sums.
// Each (row, block) partial has one writer: no atomics, deterministic.
// ---------------------------------------------------------------------------------------------------------------
template <bool SP, bool RS>
__global__ void __launch_bounds__(LayerCfg::NT) k_fc1(const uint8_t *__restrict__ h8, const float *__restrict__ hs,
                                                     int lds, const uint8_t *__restrict__ w,
                                                     const uint32_t *__restrict__ wx,
                                                     const float *__restrict__ ws, uint8_t *__restrict__ m8,
                                                     float *__restrict__ ms, float *__restrict__ stat,
                                                     const float *__restrict__ rs, int rows)
{
    using C = LayerCfg;
    constexpr int NP = C::TN / 2;                        // SwiGLU tile pairs per wave (16 units each)
    __shared__ __attribute__((aligned(16))) uint8_t smem[LAYER_SMEM];
    static_assert(C::BM * 8 % C::NT == 0, "packing items split evenly over the threads");
    int m0, n0, wm0, wn0;
    layer_tile<C>(rows, 2 * XT_HIDP, m0, n0);
    args_resident(m8, ms, stat, lds, rows);
    if constexpr (RS) args_resident(rs);
    // W12 rows past the last 16-unit chunk holding a real unit (2 x 2736) are zero padding
    constexpr int nlive = 2 * ((XT_HID + 15) / 16 * 16);
    // h tile [BM rows][128 units] fp32 in LDS, 16-byte chunk c of row r at chunk c ^ (r & 7)
    float *ht = (float *)smem;
    static_assert(C::BM * 128 * 4 <= LAYER_SMEM, "fc1 staging fits");
    static_assert(NP == 4, "two chunk pairs per 64-unit half");
    const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    const int ct = n0 >> 8;
    // silu(g) x, hardware reciprocal (1 ulp)
    auto swiglu = [](float gg, float xx) { return (gg * __builtin_amdgcn_rcpf(1.0f + __expf(-gg))) * xx; };
    // The transposed tile (sparse: as the sparse main loop leaves it; dense: TR): lane (g, c16) holds units
    // 64 wn + 16 p + 4 g + r (r = 0..3) of row wm0 + 16 i + c16 for tile pair p (gate tile 2p, value tile 2p + 1: the
    // same unit in the same register), so each (i, p) is one 16-byte chunk, 16 wn + 8 (p >> 1) + (4 (p & 1) + g), of a
    // row with row & 7 = c16 & 7: at tb[p & 1] + 2048 i + 32 (p >> 1) words.
    auto stage_h = [&](auto pair) {
        bs_wave_origin<C>(wm0, wn0);
        const int wn = wn0 / C::WN;
        uint32_t tb[2];
#pragma unroll
        for (int ph = 0; ph < 2; ph++)
            tb[ph] = (uint32_t)((wm0 + c16) * 128 + (16 * wn + ((4 * ph + g) ^ (c16 & 7))) * 4);
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int p = 0; p < NP; p++) {
                v4f gg, xx;
                pair(i, p, gg, xx);
                *(float4 *)(ht + tb[p & 1] + 2048 * i + 32 * (p >> 1)) =
                    make_float4(swiglu(gg[0], xx[0]), swiglu(gg[1], xx[1]), swiglu(gg[2], xx[2]), swiglu(gg[3], xx[3]));
            }
    };
    if constexpr (SP) {
        static_assert(C::LDS_SP <= LAYER_ROWSTAT, "sparse stages end before the row statistics");
        v4f accT[C::TN][C::TM];
        bs_mainloop_sp_t<C>(h8, XT_D, hs, lds, w, wx, ws, rows, 2 * XT_HIDP, XT_D, m0, n0, smem, accT, BsNoPre(),
                            nlive);
        stage_h([&](int i, int p, v4f &gg, v4f &xx) { gg = accT[2 * p][i]; xx = accT[2 * p + 1][i]; });
    } else {
        v4f acc[C::TM][C::TN];
        layer_mainloop<C, SP, BsNoPre, true>(h8, XT_D, hs, lds, w, wx, ws, rows, 2 * XT_HIDP, XT_D, m0, n0, smem, acc,
                                             BsNoPre(), nlive);
        stage_h([&](int i, int p, v4f &gg, v4f &xx) { gg = acc[i][2 * p]; xx = acc[i][2 * p + 1]; });
    }
    __syncthreads();
    // 8 consecutive threads per row, 16 consecutive units each: the row's |max| and sums over its 128 units meet in
    // a DPP tree over the 8 lanes; each thread packs its 16 units to E4M3 (one 16-byte store) and the first thread
    // of the row writes the block scale and the partial sums. Item it of a thread reads row
    // (tid >> 3) + 64 it, whose row & 7 does not depend on it: the four chunk addresses are bases plus 8192 it words.
    const __amdgpu_buffer_rsrc_t rm = buf_rsrc(m8, (uint32_t)rows * XT_HIDP);
    const int k8 = threadIdx.x & 7, r0 = threadIdx.x >> 3;
    uint32_t rb[4];
#pragma unroll
    for (int c = 0; c < 4; c++) rb[c] = (uint32_t)(r0 * 128 + ((((4 * k8 + c) ^ r0) & 7) | ((4 * k8 + c) & ~7)) * 4);
    float4 ru[4];  // RS: the per-unit multipliers of this thread's 16 units (the same units in every item)
    if constexpr (RS) {
#pragma unroll
        for (int c = 0; c < 4; c++) ru[c] = *(const float4 *)(rs + ct * 128 + 16 * k8 + 4 * c);
    }
#pragma unroll
    for (int it = 0; it < C::BM * 8 / C::NT; it++) {
        const int idx = threadIdx.x + it * C::NT, rr = idx >> 3, u0 = (idx & 7) * 16, m = m0 + rr;
        float4 v[4];
#pragma unroll
        for (int c = 0; c < 4; c++) v[c] = *(const float4 *)(ht + rb[c] + 128 * (C::NT / 8) * it);
        float amax = 0.f, s = 0.f, q = 0.f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            s += (v[c].x + v[c].y) + (v[c].z + v[c].w);
            q = __builtin_fmaf(v[c].x, v[c].x, q);
            q = __builtin_fmaf(v[c].y, v[c].y, q);
            q = __builtin_fmaf(v[c].z, v[c].z, q);
            q = __builtin_fmaf(v[c].w, v[c].w, q);
            if constexpr (RS) {  // the sums are over h itself, the packed operand is h rs (eva_kernels.cu:258-264)
                v[c].x *= ru[c].x;
                v[c].y *= ru[c].y;
                v[c].z *= ru[c].z;
                v[c].w *= ru[c].w;
            }
            amax = __builtin_fmaxf(__builtin_fmaxf(amax, __builtin_fabsf(v[c].x)), __builtin_fabsf(v[c].y));  // v_max3
            amax = __builtin_fmaxf(__builtin_fmaxf(amax, __builtin_fabsf(v[c].z)), __builtin_fabsf(v[c].w));
        }
        amax = row8_absmax(amax);
        s = row8_sum(s);
        q = row8_sum(q);
        const float sc = block_scale(amax), inv = block_scale_inv(sc);
        uint32_t w4[4];
#pragma unroll
        for (int c = 0; c < 4; c++) w4[c] = e4_pack4_scaled(v[c].x * inv, v[c].y * inv, v[c].z * inv, v[c].w * inv);
        const v4u o = {w4[0], w4[1], w4[2], w4[3]};
        __builtin_amdgcn_raw_buffer_store_b128(o, rm, (int)((uint32_t)m * XT_HIDP + ct * 128 + u0), 0, 0);
        if ((idx & 7) == 0 && m < rows) {
            ms[(size_t)ct * lds + m] = sc;
            *(float2 *)(stat + ((size_t)ct * lds + m) * 2) = make_float2(s, q);
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// k_fc2: x = f16(x + rstd (acc - mean c) + d) with acc = m8 . W~^T (W~ = W2 diag(gamma), c = W~ 1 from the packed
// W~, d = W2 beta), mean / rstd of the SwiGLU row over 2730 units from k_fc1's 22 partials summed in block order:
// mean = S / 2730, var = max(Q / 2730 - mean^2, 0), rstd = 1 / sqrt(var + 1e-6) (eva_kernels.cu:300-333).
// ---------------------------------------------------------------------------------------------------------------
template <bool SP>
__global__ void __launch_bounds__(LayerCfg::NT) k_fc2(const uint8_t *__restrict__ m8, const float *__restrict__ ms,
                                                     int lds, const uint8_t *__restrict__ w,
                                                     const uint32_t *__restrict__ wx,
                                                     const float *__restrict__ ws, const float *__restrict__ stat,
                                                     const float *__restrict__ cn, const float *__restrict__ dn,
                                                     uint16_t *__restrict__ x, int rows)
{
    using C = LayerCfg;
    __shared__ __attribute__((aligned(16))) uint8_t smem[LAYER_SMEM];
    v4f acc[C::TM][C::TN];
    int m0, n0, wm0, wn0;
    layer_tile<C>(rows, XT_D, m0, n0);
    float2 *rs = (float2 *)(smem + LAYER_ROWSTAT);         // [BM rows] (rstd, -mean * rstd)
    float2 *cd = (float2 *)(smem + LAYER_ROWSTAT + 2048);  // [BN columns] (c, d)
    static_assert(C::BM * 8 <= 2048 && C::BN * 8 <= 2048, "row statistics and column terms fit their 2 KB each");
    auto rowstats = [&]() {
        if (threadIdx.x < C::BM) {
            const int m = m0 + threadIdx.x;
            float2 p[XT_HIDP / 128];
#pragma unroll
            for (int blk = 0; blk < XT_HIDP / 128; blk++)
                p[blk] = m < rows ? *(const float2 *)(stat + ((size_t)blk * lds + m) * 2) : make_float2(0.f, 0.f);
            float S = 0.f, Q = 0.f;
#pragma unroll
            for (int blk = 0; blk < XT_HIDP / 128; blk++) {
                S += p[blk].x;
                Q += p[blk].y;
            }
            const float mean = S / (float)XT_HID;
            float var = Q / (float)XT_HID - mean * mean;
            var = __builtin_fmaxf(var, 0.f);
            const float rstd = 1.0f / __builtin_sqrtf(var + XT_EPS);
            rs[threadIdx.x] = make_float2(rstd, -mean * rstd);
        } else if (threadIdx.x < C::BM + C::BN) {
            const int n = n0 + threadIdx.x - C::BM;
            cd[threadIdx.x - C::BM] = make_float2(cn[n], dn[n]);
        }
    };
    args_resident(x, stat, cn, dn, lds, rows);
    static_assert(C::BM + C::BN <= C::NT, "one thread per row statistic and per column term");
    const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    // The transposed tile (sparse: as the sparse main loop leaves it; dense: TR): lane (g, c16) holds row
    // wm0 + 16 im + c16 (one row statistic per m tile) and columns wn0 + 16 jn + 4 g + r (four column terms, 32 bytes
    // of cd, per n tile). The fold is applied as the residual update parks the tile.
    float2 st[C::TM];
    auto fold = [&](v4f v, int jn, int im) {
        const float4 *cq = (const float4 *)(cd + wn0 + 16 * jn + 4 * g);
        const float4 c01 = cq[0], c23 = cq[1];  // (c, d) of columns 4 g + 0 .. 3
        v[0] = __builtin_fmaf(st[im].x, v[0], __builtin_fmaf(st[im].y, c01.x, c01.y));
        v[1] = __builtin_fmaf(st[im].x, v[1], __builtin_fmaf(st[im].y, c01.z, c01.w));
        v[2] = __builtin_fmaf(st[im].x, v[2], __builtin_fmaf(st[im].y, c23.x, c23.y));
        v[3] = __builtin_fmaf(st[im].x, v[3], __builtin_fmaf(st[im].y, c23.z, c23.w));
        return v;
    };
    if constexpr (SP) {
        static_assert(C::LDS_SP <= LAYER_ROWSTAT, "sparse stages end before the row statistics");
        v4f accT[C::TN][C::TM];
        bs_mainloop_sp_t<C>(m8, XT_HIDP, ms, lds, w, wx, ws, rows, XT_D, XT_HIDP, m0, n0, smem, accT, rowstats);
        bs_wave_origin<C>(wm0, wn0);
#pragma unroll
        for (int im = 0; im < C::TM; im++) st[im] = rs[wm0 + 16 * im + c16];
        residual_add_t<C>(smem, [&](int jn, int im) { return fold(accT[jn][im], jn, im); }, x, m0 + wm0, n0 + wn0,
                          rows);
    } else {
        layer_mainloop<C, SP, decltype(rowstats), true>(m8, XT_HIDP, ms, lds, w, wx, ws, rows, XT_D, XT_HIDP, m0, n0,
                                                       smem, acc, rowstats);
        bs_wave_origin<C>(wm0, wn0);
#pragma unroll
        for (int im = 0; im < C::TM; im++) st[im] = rs[wm0 + 16 * im + c16];
        residual_add_t<C>(smem, [&](int jn, int im) { return fold(acc[im][jn], jn, im); }, x, m0 + wm0, n0 + wn0,
                          rows);
    }
}

// ---------------------------------------------------------------------------------------------------------------
// k_head: out [nb][nt] = sigmoid(hb[n] + sum_kb ps[kb][m] hs[kb][n] sum_{k in kb} pq[m][k] hq[n][k])
// (kern_common.cuh:679-727 k_headmv, here an FP8 GEMM). The head rows carry 1x128 scales of their own (planes
// hs [8][ldh], as activations do), so every row is packed, and repacked by eva_head_put, independently of all others.
// The head is a weight stream (nt x 1 KB) against at most 128 input rows: one block per 64 output columns and 64 rows,
// 4 waves, wave w owning columns n0 + 16 w .. + 15. A wave issues the loads of all eight K blocks' weight fragments
// and scales before its first matrix instruction (one memory round trip for the stream instead of eight), then runs
// only the row tiles of 16 that hold input rows (a batch of 16 runs one of the four). Fragments come straight from L2
// into registers; descriptors that end at row nb of pq and row nt of hq load zero past them. Each output's K blocks
// are promoted in order, so a row's scores do not depend on the batch around it.
// ---------------------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) k_head(const uint8_t *__restrict__ pq, const float *__restrict__ ps, int lds,
                                              const uint8_t *__restrict__ hq, const float *__restrict__ hs, int ldh,
                                              const float *__restrict__ hb, float *__restrict__ out, int nb, int nt)
{
    constexpr int KB = XT_D / 128;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    const int n0 = blockIdx.x * 64 + 16 * w, m0 = blockIdx.y * 64;
    const __amdgpu_buffer_rsrc_t ra = buf_rsrc(pq, (uint32_t)nb * XT_D), rw = buf_rsrc(hq, (uint32_t)nt * XT_D);
    const int nl = n0 + c16;                                  // weight row of this lane's B fragment, output column
    const int ncl = nl < nt ? nl : nt - 1;                    // clamped for the scale and bias reads
    v8i b[KB];
    float swv[KB];
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
        const uint32_t ko = (uint32_t)kb * 128u + 16u * g;
        const v4u blo = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)((uint32_t)nl * XT_D + ko), 0, 0);
        const v4u bhi = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)((uint32_t)nl * XT_D + ko + 64u), 0, 0);
        b[kb] = v8i{(int)blo[0], (int)blo[1], (int)blo[2], (int)blo[3], (int)bhi[0], (int)bhi[1], (int)bhi[2], (int)bhi[3]};
        swv[kb] = hs[(size_t)kb * ldh + ncl];
    }
    const int ntile = (nb - m0 + 15) >> 4;                    // row tiles holding input rows (block-uniform, >= 1)
    const float bias = hb[ncl];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (i >= ntile) break;
        v8i a[KB];
        float sa[KB][4];
        const uint32_t ar = (uint32_t)(m0 + 16 * i + c16) * XT_D;
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            const uint32_t ko = (uint32_t)kb * 128u + 16u * g;
            const v4u alo = __builtin_amdgcn_raw_buffer_load_b128(ra, (int)(ar + ko), 0, 0);
            const v4u ahi = __builtin_amdgcn_raw_buffer_load_b128(ra, (int)(ar + ko + 64u), 0, 0);
            a[kb] = v8i{(int)alo[0], (int)alo[1], (int)alo[2], (int)alo[3], (int)ahi[0], (int)ahi[1], (int)ahi[2], (int)ahi[3]};
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + 16 * i + 4 * g + r;
                sa[kb][r] = m < nb ? ps[(size_t)kb * lds + m] : 0.f;
            }
        }
        v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            const v4f p = mfma_e4m3_16x16x128(a[kb], b[kb]);
#pragma unroll
            for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(p[r], sa[kb][r] * swv[kb], acc[r]);
        }
        if (nl < nt)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + 16 * i + 4 * g + r;
                if (m < nb) out[(size_t)m * nt + nl] = 1.0f / (1.0f + __expf(-(acc[r] + bias)));
            }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// k_pe: patch embedding in fp16 with fp32 accumulation (v_mfma_f32_16x16x32_f16) and the position add fused
// (k_pe + k_embed, eva_kernels.cu:21-33, 126-130): x[1025 b + 1 + p] = f16(in[1024 b + p] . pe^T + pos[1 + p]),
// x[1025 b] = f16(pos[0]) (pos carries cls and the conv bias, export_eva.py:76-80). Block 128 patches x 128
// columns, 4 waves of 64 x 64, K = 592 in steps of 64 halves (the last step holds 16; the rest is zeroed).
// ---------------------------------------------------------------------------------------------------------------
// PX: the PixAI patch GEMM (px_kernels.cu:133-138 k_ppe) instead: x[m] = f16(in[m] . pe^T) for window-major token rows
// m (no cls, no position: k_px_pembed adds it before its LayerNorm), rows a multiple of 128.
template <bool PX>
__global__ void __launch_bounds__(256) k_pe(const uint16_t *__restrict__ in, const uint16_t *__restrict__ pe,
                                            const float *__restrict__ pos, uint16_t *__restrict__ x, int nb)
{
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * 128 * 128];  // A | B tile of one K step
    const int m0 = blockIdx.y * 128, n0 = blockIdx.x * 128, t = threadIdx.x;
    const int lane = t & 63, w = t >> 6, g = lane >> 4, r16 = lane & 15;
    const int wm0 = (w >> 1) * 64, wn0 = (w & 1) * 64;
    v4f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    // stage: 128 rows x 8 chunks of 8 halves for A and B; chunks past column 592 are zero. The next K step's chunks
    // are loaded into registers while the current step's MFMAs run.
    uint4 va[4], vb[4];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int it = 0; it < 4; it++) {
            const int idx = t + 256 * it, row = idx >> 3, ch = idx & 7, col = k0 + 8 * ch;
            va[it] = vb[it] = make_uint4(0, 0, 0, 0);
            if (col < XT_K0P) {
                va[it] = *(const uint4 *)(in + (size_t)(m0 + row) * XT_K0P + col);
                vb[it] = *(const uint4 *)(pe + (size_t)(n0 + row) * XT_K0P + col);
            }
        }
    };
    fetch(0);
    for (int k0 = 0; k0 < XT_K0P; k0 += 64) {
#pragma unroll
        for (int it = 0; it < 4; it++) {
            const int idx = t + 256 * it, row = idx >> 3, ch = idx & 7;
            *(uint4 *)(smem + swz(row, ch)) = va[it];
            *(uint4 *)(smem + 128 * 128 + swz(row, ch)) = vb[it];
        }
        __syncthreads();
        if (k0 + 64 < XT_K0P) fetch(k0 + 64);
#pragma unroll
        for (int s = 0; s < 2; s++) {
            v8h a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; i++) a[i] = __builtin_bit_cast(v8h, *(const uint4 *)(smem + swz(wm0 + 16 * i + r16, 4 * s + g)));
#pragma unroll
            for (int j = 0; j < 4; j++)
                b[j] = __builtin_bit_cast(v8h, *(const uint4 *)(smem + 128 * 128 + swz(wn0 + 16 * j + r16, 4 * s + g)));
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
    const int c16 = lane & 15;
    if constexpr (PX) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                uint16_t *xr = x + (size_t)(m0 + wm0 + 16 * i + 4 * g + r) * XT_D;
#pragma unroll
                for (int j = 0; j < 4; j++) xr[n0 + wn0 + 16 * j + c16] = f2h(acc[i][j][r]);
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = m0 + wm0 + 16 * i + 4 * g + r, b = m >> 10, p = m & 1023;
            uint16_t *xr = x + ((size_t)b * XT_T + 1 + p) * XT_D;
            const float *pr = pos + (size_t)(1 + p) * XT_D;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int n = n0 + wn0 + 16 * j + c16;
                xr[n] = f2h(acc[i][j][r] + pr[n]);
            }
        }
    if ((m0 & 1023) == 0 && t < 128) {  // the first patch tile of an image also writes its cls row
        const int b = m0 >> 10, n = n0 + t;
        x[(size_t)b * XT_T * XT_D + n] = f2h(pos[n]);
    }
}

// ---------------------------------------------------------------------------------------------------------------
// C-ABI launchers
// ---------------------------------------------------------------------------------------------------------------
template <bool SP>
static int qkv_launch(const char *what, const void *h8, const float *hs, int lds, const void *w, const void *wx,
                      const float *ws, const float *cs, void *q, void *k, void *vt, int rows, void *stream)
{
    if (layer_rows_ok(what, rows, lds)) return -1;
    if (rows % XT_T) return xt_fail(what, "rows must be nb * 1025");
    if (!XT_ALIGNED(h8) || !XT_ALIGNED(w) || (SP && !wx)) return xt_fail(what, "h8 and w must be 16-byte aligned");
    hipLaunchKernelGGL(k_qkv<SP>, dim3(layer_grid(rows, 3 * XT_D, LayerCfg::BM, LayerCfg::BN)), dim3(LayerCfg::NT), 0,
                       (hipStream_t)stream, (const uint8_t *)h8, hs, lds, (const uint8_t *)w, (const uint32_t *)wx, ws,
                       cs, (uint16_t *)q, (uint16_t *)k, (uint16_t *)vt, rows);
    return xt_check(what);
}

template <bool SP>
static int oproj_launch(const char *what, const void *a8, const float *as, int lds, const void *w, const void *wx,
                        const float *ws, void *x, int rows, void *stream)
{
    if (layer_rows_ok(what, rows, lds)) return -1;
    if (!XT_ALIGNED(a8) || !XT_ALIGNED(w) || (SP && !wx)) return xt_fail(what, "a8 and w must be 16-byte aligned");
    hipLaunchKernelGGL(k_oproj<SP>, dim3(layer_grid(rows, XT_D, LayerCfg::BM, LayerCfg::BN)), dim3(LayerCfg::NT), 0,
                       (hipStream_t)stream, (const uint8_t *)a8, as, lds, (const uint8_t *)w, (const uint32_t *)wx, ws,
                       (uint16_t *)x, rows);
    return xt_check(what);
}

template <bool SP>
static int fc1_launch(const char *what, const void *h8, const float *hs, int lds, const void *w, const void *wx,
                      const float *ws, void *m8, float *ms, float *stat, const float *rs, int rows, void *stream)
{
    if (layer_rows_ok(what, rows, lds)) return -1;
    if (!XT_ALIGNED(h8) || !XT_ALIGNED(w) || !XT_ALIGNED(m8) || !XT_ALIGNED(rs) || (SP && !wx))
        return xt_fail(what, "h8, w, m8, rs must be 16-byte aligned");
    const dim3 grid(layer_grid(rows, 2 * XT_HIDP, LayerCfg::BM, LayerCfg::BN));
    if (rs)
        hipLaunchKernelGGL((k_fc1<SP, true>), grid, dim3(LayerCfg::NT), 0, (hipStream_t)stream, (const uint8_t *)h8, hs,
                           lds, (const uint8_t *)w, (const uint32_t *)wx, ws, (uint8_t *)m8, ms, stat, rs, rows);
    else
        hipLaunchKernelGGL((k_fc1<SP, false>), grid, dim3(LayerCfg::NT), 0, (hipStream_t)stream, (const uint8_t *)h8, hs,
                           lds, (const uint8_t *)w, (const uint32_t *)wx, ws, (uint8_t *)m8, ms, stat, rs, rows);
    return xt_check(what);
}

template <bool SP>
static int fc2_launch(const char *what, const void *m8, const float *ms, int lds, const void *w, const void *wx,
                      const float *ws, const float *stat, const float *cn, const float *dn, void *x, int rows,
                      void *stream)
{
    if (layer_rows_ok(what, rows, lds)) return -1;
    if (!XT_ALIGNED(m8) || !XT_ALIGNED(w) || (SP && !wx)) return xt_fail(what, "m8 and w must be 16-byte aligned");
    hipLaunchKernelGGL(k_fc2<SP>, dim3(layer_grid(rows, XT_D, LayerCfg::BM, LayerCfg::BN)), dim3(LayerCfg::NT), 0,
                       (hipStream_t)stream, (const uint8_t *)m8, ms, lds, (const uint8_t *)w, (const uint32_t *)wx, ws,
                       stat, cn, dn, (uint16_t *)x, rows);
    return xt_check(what);
}

extern "C" int eva_k_qkv(const void *h8, const float *hs, int lds, const void *w, const float *ws, const float *cs,
                         void *q, void *k, void *vt, int rows, void *stream)
{
    return qkv_launch<false>("eva_k_qkv", h8, hs, lds, w, nullptr, ws, cs, q, k, vt, rows, stream);
}

extern "C" int eva_k_oproj(const void *a8, const float *as, int lds, const void *w, const float *ws, void *x, int rows,
                           void *stream)
{
    return oproj_launch<false>("eva_k_oproj", a8, as, lds, w, nullptr, ws, x, rows, stream);
}

extern "C" int eva_k_fc1(const void *h8, const float *hs, int lds, const void *w, const float *ws, void *m8, float *ms,
                         float *stat, int rows, void *stream)
{
    return fc1_launch<false>("eva_k_fc1", h8, hs, lds, w, nullptr, ws, m8, ms, stat, nullptr, rows, stream);
}

extern "C" int eva_k_fc1_rs(const void *h8, const float *hs, int lds, const void *w, const float *ws, void *m8,
                            float *ms, float *stat, const float *rs, int rows, void *stream)
{
    if (!rs) return xt_fail("eva_k_fc1_rs", "rs must not be NULL");
    return fc1_launch<false>("eva_k_fc1_rs", h8, hs, lds, w, nullptr, ws, m8, ms, stat, rs, rows, stream);
}

extern "C" int eva_k_fc2(const void *m8, const float *ms, int lds, const void *w, const float *ws, const float *stat,
                         const float *cn, const float *dn, void *x, int rows, void *stream)
{
    return fc2_launch<false>("eva_k_fc2", m8, ms, lds, w, nullptr, ws, stat, cn, dn, x, rows, stream);
}

extern "C" int eva_k_qkv_sp(const void *h8, const float *hs, int lds, const void *vals, const void *idx,
                            const float *ws, const float *cs, void *q, void *k, void *vt, int rows, void *stream)
{
    return qkv_launch<true>("eva_k_qkv_sp", h8, hs, lds, vals, idx, ws, cs, q, k, vt, rows, stream);
}

extern "C" int eva_k_oproj_sp(const void *a8, const float *as, int lds, const void *vals, const void *idx,
                              const float *ws, void *x, int rows, void *stream)
{
    return oproj_launch<true>("eva_k_oproj_sp", a8, as, lds, vals, idx, ws, x, rows, stream);
}

extern "C" int eva_k_fc1_sp(const void *h8, const float *hs, int lds, const void *vals, const void *idx,
                            const float *ws, void *m8, float *ms, float *stat, int rows, void *stream)
{
    return fc1_launch<true>("eva_k_fc1_sp", h8, hs, lds, vals, idx, ws, m8, ms, stat, nullptr, rows, stream);
}

extern "C" int eva_k_fc1_rs_sp(const void *h8, const float *hs, int lds, const void *vals, const void *idx,
                               const float *ws, void *m8, float *ms, float *stat, const float *rs, int rows,
                               void *stream)
{
    if (!rs) return xt_fail("eva_k_fc1_rs_sp", "rs must not be NULL");
    return fc1_launch<true>("eva_k_fc1_rs_sp", h8, hs, lds, vals, idx, ws, m8, ms, stat, rs, rows, stream);
}

extern "C" int eva_k_fc2_sp(const void *m8, const float *ms, int lds, const void *vals, const void *idx,
                            const float *ws, const float *stat, const float *cn, const float *dn, void *x, int rows,
                            void *stream)
{
    return fc2_launch<true>("eva_k_fc2_sp", m8, ms, lds, vals, idx, ws, stat, cn, dn, x, rows, stream);
}

extern "C" int eva_k_head(const void *pq, const float *ps, int lds, const void *w, const float *ws, int ldw,
                          const float *hb, float *out, int nb, int nt, void *stream)
{
    if (nb <= 0 || nt <= 0 || lds < nb || ldw < nt || nb > EVA_NBMAX || nt > (1 << 20))
        return xt_fail("eva_k_head", "bad shape (0 < nb <= 128, 0 < nt <= 2^20, lds >= nb, ldw >= nt)");
    if (!XT_ALIGNED(pq) || !XT_ALIGNED(w)) return xt_fail("eva_k_head", "pq and w must be 16-byte aligned");
    hipLaunchKernelGGL(k_head, dim3((nt + 63) / 64, (nb + 63) / 64), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t *)pq, ps, lds, (const uint8_t *)w, ws, ldw, hb, out, nb, nt);
    return xt_check("eva_k_head");
}

extern "C" int eva_k_pe(const void *in, const void *pe, const float *pos, void *x, int nb, void *stream)
{
    if (nb <= 0) return xt_fail("eva_k_pe", "nb must be positive");
    if (!XT_ALIGNED(in) || !XT_ALIGNED(pe)) return xt_fail("eva_k_pe", "in and pe must be 16-byte aligned");
    hipLaunchKernelGGL(k_pe<false>, dim3(XT_D / 128, nb * XT_NP / 128), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t *)in, (const uint16_t *)pe, pos, (uint16_t *)x, nb);
    return xt_check("eva_k_pe");
}

extern "C" int px_k_pe(const void *in, const void *pe, void *x, int rows, void *stream)
{
    if (rows <= 0 || rows % 128) return xt_fail("px_k_pe", "rows must be a positive multiple of 128 (an even batch)");
    if (!XT_ALIGNED(in) || !XT_ALIGNED(pe)) return xt_fail("px_k_pe", "in and pe must be 16-byte aligned");
    hipLaunchKernelGGL(k_pe<true>, dim3(XT_D / 128, rows / 128), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t *)in, (const uint16_t *)pe, (const float *)nullptr, (uint16_t *)x, 0);
    return xt_check("px_k_pe");
}
