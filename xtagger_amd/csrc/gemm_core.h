// gemm_core.h - block-scaled E4M3 GEMM main loop for gfx950 (the role of the reference's gemm8,
// src/engine/kern_common.cuh:271-356, generalised from one per-tensor alpha to per-block scales).
//
//   acc[m][n] = sum_kb sa[kb][m] * sw[n / 128][kb] * sum_{k in kb} A[m][k] * W[n][k]
//
// A [M][lda] E4M3 bytes (activations, 1x128 scales sa [K/128][lds]), W [N][K] E4M3 bytes (weights, 128x128 scales
// sw [ceil(N/128)][K/128], rows padded with zeros to a multiple of 128). K % 128 == 0.
//
// CDNA4 mapping: one K step = one 128-wide scale block = one v_mfma_f32_16x16x128_f8f6f4 per 16x16 output tile, so
// the per-block partial comes out of the matrix core whole and is promoted with one fma per accumulator
// (acc = fma(partial, sa * sw, acc)). Tiles of BM x 128 / BN x 128 bytes are staged through LDS, double-buffered
// with register prefetch; 16-byte chunk c of LDS row r lives at chunk c ^ (r & 7), so the 16 lanes that read one
// chunk column of 16 consecutive rows hit 8 distinct bank groups per half. Waves are laid out (BM/WM) x (BN/WN);
// each owns a WM x WN sub-tile of 16x16 MFMA tiles. A wave's WN columns sit inside one 128-column weight block.
#pragma once
#include "xt_common.h"

template <int BM, int BN, int WM, int WN>
struct BsCfg {
    static constexpr int NWM = BM / WM;
    static constexpr int NWN = BN / WN;
    static constexpr int NW = NWM * NWN;
    static constexpr int NT = NW * 64;
    static constexpr int TM = WM / 16;
    static constexpr int TN = WN / 16;
    static constexpr int A_BYTES = BM * 128;
    static constexpr int B_BYTES = BN * 128;
    static constexpr int S_BYTES = BM * 4;
    static constexpr int STAGE = A_BYTES + B_BYTES + S_BYTES;
    static constexpr int LDS = 2 * STAGE;
    static constexpr int CA = BM * 8 / NT;  // A chunks per thread per stage
    static constexpr int CB = BN * 8 / NT;  // B chunks per thread per stage
    static_assert(BM * 8 % NT == 0 && BN * 8 % NT == 0, "tile / thread mismatch");
    static_assert(WN <= 128 && 128 % WN == 0, "a wave's columns must sit in one weight block");
    static_assert(BM <= NT, "one scale per thread");
};

__device__ __forceinline__ uint32_t swz(int row, int chunk) { return (uint32_t)(row * 128 + ((chunk ^ (row & 7)) << 4)); }

template <int BM, int BN, int WM, int WN>
struct BsLoader {
    using C = BsCfg<BM, BN, WM, WN>;
    uint4 ra[C::CA];
    uint4 rb[C::CB];
    float rs;

    __device__ __forceinline__ void load(const uint8_t *__restrict__ A, int lda, const float *__restrict__ sa, int lds,
                                         const uint8_t *__restrict__ W, int K, int M, int m0, int n0, int kb)
    {
        const int t = threadIdx.x, c = t & 7, r0 = t >> 3;
#pragma unroll
        for (int i = 0; i < C::CA; i++) {
            const int row = r0 + (C::NT / 8) * i, gm = m0 + row;
            ra[i] = gm < M ? *(const uint4 *)(A + (size_t)gm * lda + kb * 128 + c * 16) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < C::CB; i++) {
            const int row = r0 + (C::NT / 8) * i;
            rb[i] = *(const uint4 *)(W + (size_t)(n0 + row) * K + kb * 128 + c * 16);
        }
        rs = (t < BM && m0 + t < M) ? sa[(size_t)kb * lds + m0 + t] : 0.0f;
    }

    __device__ __forceinline__ void store(uint8_t *stage)
    {
        const int t = threadIdx.x, c = t & 7, r0 = t >> 3;
#pragma unroll
        for (int i = 0; i < C::CA; i++) *(uint4 *)(stage + swz(r0 + (C::NT / 8) * i, c)) = ra[i];
#pragma unroll
        for (int i = 0; i < C::CB; i++) *(uint4 *)(stage + C::A_BYTES + swz(r0 + (C::NT / 8) * i, c)) = rb[i];
        if (t < BM) ((float *)(stage + C::A_BYTES + C::B_BYTES))[t] = rs;
    }
};

// 32 bytes of LDS row `row` for lane group g (logical chunks 2g, 2g+1) as an MFMA operand. A and B use the same
// (lane group, byte) -> k map, so the product sums over every k of the block exactly once.
__device__ __forceinline__ v8i ld_frag(const uint8_t *tile, int row, int g)
{
    uint4 lo = *(const uint4 *)(tile + swz(row, 2 * g));
    uint4 hi = *(const uint4 *)(tile + swz(row, 2 * g + 1));
    v8i v;
    v[0] = (int)lo.x; v[1] = (int)lo.y; v[2] = (int)lo.z; v[3] = (int)lo.w;
    v[4] = (int)hi.x; v[5] = (int)hi.y; v[6] = (int)hi.z; v[7] = (int)hi.w;
    return v;
}

// Main loop. On return acc[i][j][r] holds output row m0 + wm0 + 16 i + 4 (lane >> 4) + r, column
// n0 + wn0 + 16 j + (lane & 15), where (wm0, wn0) = bs_wave_origin(). The block is synchronised and the shared
// memory is free for the epilogue.
template <int BM, int BN, int WM, int WN>
__device__ __forceinline__ void bs_wave_origin(int &wm0, int &wn0)
{
    using C = BsCfg<BM, BN, WM, WN>;
    const int w = threadIdx.x >> 6;
    wm0 = (w / C::NWN) * WM;
    wn0 = (w % C::NWN) * WN;
}

template <int BM, int BN, int WM, int WN>
__device__ __forceinline__ void bs_mainloop(const uint8_t *__restrict__ A, int lda, const float *__restrict__ sa,
                                            int lds, const uint8_t *__restrict__ W, const float *__restrict__ sw,
                                            int M, int K, int m0, int n0, uint8_t *smem,
                                            v4f (&acc)[BsCfg<BM, BN, WM, WN>::TM][BsCfg<BM, BN, WM, WN>::TN])
{
    using C = BsCfg<BM, BN, WM, WN>;
    BsLoader<BM, BN, WM, WN> ld;
    const int lane = threadIdx.x & 63, g = lane >> 4, r16 = lane & 15;
    const int KB = K >> 7;
    int wm0, wn0;
    bs_wave_origin<BM, BN, WM, WN>(wm0, wn0);
    const float *swp = sw + (size_t)((n0 + wn0) >> 7) * KB;

#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int j = 0; j < C::TN; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    ld.load(A, lda, sa, lds, W, K, M, m0, n0, 0);
    ld.store(smem);
    __syncthreads();
    for (int kb = 0; kb < KB; kb++) {
        uint8_t *st = smem + (kb & 1) * C::STAGE;
        if (kb + 1 < KB) ld.load(A, lda, sa, lds, W, K, M, m0, n0, kb + 1);
        const float swv = swp[kb];
        const uint8_t *ta = st, *tb = st + C::A_BYTES;
        const float *ts = (const float *)(st + C::A_BYTES + C::B_BYTES);
        v8i b[C::TN];
#pragma unroll
        for (int j = 0; j < C::TN; j++) b[j] = ld_frag(tb, wn0 + 16 * j + r16, g);
#pragma unroll
        for (int i = 0; i < C::TM; i++) {
            const v8i a = ld_frag(ta, wm0 + 16 * i + r16, g);
            const float4 s4 = *(const float4 *)(ts + wm0 + 16 * i + 4 * g);
            const float sc0 = s4.x * swv, sc1 = s4.y * swv, sc2 = s4.z * swv, sc3 = s4.w * swv;
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                const v4f p = mfma_e4m3_16x16x128(a, b[j]);
                acc[i][j][0] = __builtin_fmaf(p[0], sc0, acc[i][j][0]);
                acc[i][j][1] = __builtin_fmaf(p[1], sc1, acc[i][j][1]);
                acc[i][j][2] = __builtin_fmaf(p[2], sc2, acc[i][j][2]);
                acc[i][j][3] = __builtin_fmaf(p[3], sc3, acc[i][j][3]);
            }
        }
        if (kb + 1 < KB) ld.store(smem + ((kb + 1) & 1) * C::STAGE);
        __syncthreads();
    }
}
