// quant.hip - E4M3 packing with per-block fp32 scales (activations 1x128, weights 128x128) and the standalone
// block-scaled GEMM. Reference roles: q2 / st4 / st8h (src/engine/kern_common.cuh:97-128) for activations,
// fp8() (src/tools/export_eva.py:64-66) for weights, gemm8 (kern_common.cuh:271-356) for the GEMM.
#include "gemm_core.h"
#include "xt_abi.h"

// ---- activations: x [M][ldx] (bf16, fp32 or fp16) -> q [M][ldq] E4M3, s [K/128][lds] ----
// One thread per 8 consecutive elements; the 16 threads of one 128-element block are 16 aligned lanes.
template <typename TIn>
__device__ __forceinline__ void load8(const TIn *p, float *v);
template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t *p, float *v)
{
    const uint4 u = *(const uint4 *)p;
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}
template <>
__device__ __forceinline__ void load8<_Float16>(const _Float16 *p, float *v)
{
    const v8h h = *(const v8h *)p;
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = (float)h[i];
}
template <>
__device__ __forceinline__ void load8<float>(const float *p, float *v)
{
    const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

template <typename TIn>
__global__ void __launch_bounds__(256) k_quant_act(const TIn *__restrict__ x, int ldx, int M, int K,
                                                   uint8_t *__restrict__ q, int ldq, float *__restrict__ s, int lds)
{
    const int cpr = K >> 3;  // 8-element chunks per row
    const long total = (long)M * cpr;
    for (long t = (long)blockIdx.x * 256 + threadIdx.x; t < total; t += (long)gridDim.x * 256) {
        // the 16 lanes of a block share every trip: total and the stride are multiples of 16
        const int row = (int)(t / cpr), ch = (int)(t - (long)row * cpr);
        float v[8], amax = 0.f;
        load8<TIn>(x + (size_t)row * ldx + ch * 8, v);
#pragma unroll
        for (int i = 0; i < 8; i++) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));
        amax = row16_absmax(amax);  // the 16 lanes of the block: one DPP row, all active together
        const float sc = block_scale(amax), inv = block_scale_inv(sc);
        uint2 o;
        o.x = e4_pack4_scaled(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
        o.y = e4_pack4_scaled(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv);
        *(uint2 *)(q + (size_t)row * ldq + ch * 8) = o;
        if ((ch & 15) == 0) s[(size_t)(ch >> 4) * lds + row] = sc;
    }
}

// ---- weights: w [N][K] fp32 -> q [ceil(N/128)*128][K] E4M3 (pad rows zero), s [ceil(N/128)][K/128] ----
// One 256-thread block per 128 x 128 block: 64 elements per thread, |max| through LDS, then q = sat_rne(w / s).
__global__ void __launch_bounds__(256) k_quant_w(const float *__restrict__ w, int N, int K, uint8_t *__restrict__ q,
                                                 float *__restrict__ s)
{
    __shared__ float red[4];
    const int kb = blockIdx.x, nb = blockIdx.y, KB = K >> 7;
    const int t = threadIdx.x, c = t & 15, r0 = t >> 4;  // 16 threads x 8 columns cover a 128-wide row
    float amax = 0.f;
    for (int r = r0; r < 128; r += 16) {
        const int n = nb * 128 + r;
        if (n < N) {
            float v[8];
            load8<float>(w + (size_t)n * K + kb * 128 + c * 8, v);
#pragma unroll
            for (int i = 0; i < 8; i++) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));
        }
    }
    amax = wave_max(amax);
    if ((t & 63) == 0) red[t >> 6] = amax;
    __syncthreads();
    amax = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
    const float sc = block_scale(amax);
    if (t == 0) s[(size_t)nb * KB + kb] = sc;
    for (int r = r0; r < 128; r += 16) {
        const int n = nb * 128 + r;
        uint2 o = make_uint2(0, 0);
        if (n < N) {
            float v[8];
            load8<float>(w + (size_t)n * K + kb * 128 + c * 8, v);
            o.x = e4_pack4(v[0] / sc, v[1] / sc, v[2] / sc, v[3] / sc);
            o.y = e4_pack4(v[4] / sc, v[5] / sc, v[6] / sc, v[7] / sc);
        }
        *(uint2 *)(q + (size_t)n * K + kb * 128 + c * 8) = o;
    }
}

// ---- encoder check: E4M3 of the fp32 bit patterns first .. first + count - 1 ----
__global__ void __launch_bounds__(256) k_e4m3_bits(uint32_t first, uint32_t count, uint8_t *__restrict__ out)
{
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < count; i += gridDim.x * 256u)
        out[i] = (uint8_t)e4_pack2(__uint_as_float(first + i), 0.f);
}

// ---- block-scale rule check: block_scale (which 0) or block_scale_inv (which 1) of the fp32 bit patterns
// first .. first + count - 1, as bit patterns ----
__global__ void __launch_bounds__(256) k_scale_bits(uint32_t first, uint32_t count, int which, uint32_t *__restrict__ out)
{
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < count; i += gridDim.x * 256u) {
        const float x = __uint_as_float(first + i);
        out[i] = __float_as_uint(which ? block_scale_inv(x) : block_scale(x));
    }
}

// ---- standalone block-scaled GEMM: C [M][ldc] = bf16 or fp32 of the block-scaled product ----
// bf16: each wave parks 64 x 64 fp32 of its tile in its own LDS slice (row stride 68 floats, conflict-free), then
// every lane rounds 8 consecutive columns to bf16 (RNE) and writes them with one 16-byte store through a descriptor
// that ends at row M (rows past it are dropped). ldc and N multiples of 8 and a 16-byte aligned C take that path; other
// shapes store element by element. fp32 (the parity build) stores straight from the accumulators.
constexpr int GEMM_SLICE = 64 * 68 * 4;
template <class C>
constexpr int gemm_smem()
{
    return C::LDS > C::NW * GEMM_SLICE ? (C::LDS > C::LDS_SP ? C::LDS : C::LDS_SP)
                                       : (C::NW * GEMM_SLICE > C::LDS_SP ? C::NW * GEMM_SLICE : C::LDS_SP);
}

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// SP: W holds the 2:4 values and WX the indices of the pack24 layout (bs_mainloop_sp); otherwise W is dense, WX unused.
template <class C, int OUT, bool SP>  // OUT 0: bf16, 1: fp32
__global__ void __launch_bounds__(C::NT) k_gemm(const uint8_t *__restrict__ A, int lda, const float *__restrict__ sa,
                                               int lds, const uint8_t *__restrict__ W, const uint32_t *__restrict__ WX,
                                               const float *__restrict__ sw, void *__restrict__ Cp, int ldc, int M,
                                               int N, int K)
{
    static_assert(C::TM == 4 && C::TN % 4 == 0, "64-row wave tiles, whole 64-column passes");
    __shared__ __attribute__((aligned(16))) uint8_t smem[gemm_smem<C>()];
    v4f acc[C::TM][C::TN];
    int tm, tn;
    tile_of_block((M + C::BM - 1) / C::BM, (N + C::BN - 1) / C::BN, M % C::BM != 0, tm, tn);
    const int m0 = tm * C::BM, n0 = tn * C::BN, lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    const int Npad = (N + 127) & ~127;
    args_resident(Cp, ldc, N, M, lds);
    // the tile transposed (acc[i][j][r]: row m0 + wm0 + 16 i + c16, column n0 + wn0 + 16 j + 4 g + r): the sparse
    // loop's own layout, and the dense loop's with TR
    if constexpr (SP) {
        v4f accT[C::TN][C::TM];
        bs_mainloop_sp_t<C, BsNoPre, false>(A, lda, sa, lds, W, WX, sw, M, Npad, K, m0, n0, smem, accT);
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int j = 0; j < C::TN; j++) acc[i][j] = accT[j][i];
    } else {
        bs_mainloop<C, BsNoPre, false, true>(A, lda, sa, lds, W, sw, M, Npad, K, m0, n0, smem, acc);
    }
    int wm0, wn0;
    bs_wave_origin<C>(wm0, wn0);
    if (OUT == 1) {
        const bool v4ok = (ldc | N) % 4 == 0 && (((uintptr_t)Cp) & 15) == 0;  // whole 16-byte column quads
#pragma unroll
        for (int i = 0; i < C::TM; i++) {
            const int row = m0 + wm0 + 16 * i + c16;
            if (row >= M) continue;
            float *crow = (float *)Cp + (size_t)row * ldc;
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                const int col = n0 + wn0 + 16 * j + 4 * g;
                if (v4ok) {
                    if (col < N) *(float4 *)(crow + col) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (col + r < N) crow[col + r] = acc[i][j][r];
                }
            }
        }
        return;
    }
    uint16_t *Cb = (uint16_t *)Cp;
    if ((ldc | N) % 8 != 0 || (((uintptr_t)Cp) & 15)) {  // general shapes: one element per store
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                const int row = m0 + wm0 + 16 * i + c16;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int col = n0 + wn0 + 16 * j + 4 * g + r;
                    if (row < M && col < N) Cb[(size_t)row * ldc + col] = f2bf(acc[i][j][r]);
                }
            }
        return;
    }
    float *tr = (float *)(smem + (threadIdx.x >> 6) * GEMM_SLICE);
    const __amdgpu_buffer_rsrc_t rc = buf_rsrc(Cp, (uint32_t)M * (uint32_t)ldc * 2u);
    const int rs = lane >> 3, ch = lane & 7;
#pragma unroll
    for (int pass = 0; pass < C::TN / 4; pass++) {
        if (pass) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the previous pass's slice reads are done
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const v4f v = acc[i][4 * pass + j];
                *(float4 *)(tr + (16 * i + c16) * 68 + 16 * j + 4 * g) = make_float4(v[0], v[1], v[2], v[3]);
            }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slice is the wave's own: no block barrier needed
        const int col = n0 + wn0 + 64 * pass + 8 * ch;
#pragma unroll
        for (int it = 0; it < 8; it++) {
            const int rr = 8 * it + rs;
            const float4 a = *(const float4 *)(tr + rr * 68 + 8 * ch), b = *(const float4 *)(tr + rr * 68 + 8 * ch + 4);
            const v4u o = {f2bf(a.x) | (uint32_t)f2bf(a.y) << 16, f2bf(a.z) | (uint32_t)f2bf(a.w) << 16,
                           f2bf(b.x) | (uint32_t)f2bf(b.y) << 16, f2bf(b.z) | (uint32_t)f2bf(b.w) << 16};
            if (col < N)
                __builtin_amdgcn_raw_buffer_store_b128(o, rc, (int)(((uint32_t)(m0 + wm0 + rr) * (uint32_t)ldc + col) * 2u), 0, 0);
        }
    }
}

typedef BsCfg<256, 256, 4, 2, 2> GemmBig;    // 8 waves of 64 x 128, 2 stages: once the tiles fill the 256 CUs
typedef BsCfg<128, 128, 2, 2, 2> GemmMid;    // 4 waves of 64 x 64, 2 stages, two blocks per CU: small M

// ---------------------------------------------------------------------------------------------------------------
// C-ABI launchers
// ---------------------------------------------------------------------------------------------------------------
static int grid_for(long threads)
{
    long b = (threads + 255) / 256;
    return (int)(b < 1 ? 1 : b > 65535 ? 65535 : b);
}

extern "C" int eva_k_quant_act(const void *x, int in_kind, int ldx, int M, int K, void *q, int ldq, float *s, int lds,
                               void *stream)
{
    if (M < 0 || K % 128 || ldx < K || ldq < K || lds < M || in_kind < 0 || in_kind > 2 || ldx % 8 || ldq % 8)
        return xt_fail("eva_k_quant_act",
                       "bad shape (K % 128, ldx >= K, ldq >= K, lds >= M, ldx and ldq multiples of 8, in_kind 0..2)");
    if (((uintptr_t)x | (uintptr_t)q) & 15) return xt_fail("eva_k_quant_act", "x and q must be 16-byte aligned");
    if (!M) return 0;
    const long thr = (long)M * (K / 8);
    if (in_kind == 0)
        hipLaunchKernelGGL(k_quant_act<uint16_t>, dim3(grid_for(thr)), dim3(256), 0, (hipStream_t)stream,
                           (const uint16_t *)x, ldx, M, K, (uint8_t *)q, ldq, s, lds);
    else if (in_kind == 1)
        hipLaunchKernelGGL(k_quant_act<float>, dim3(grid_for(thr)), dim3(256), 0, (hipStream_t)stream, (const float *)x,
                           ldx, M, K, (uint8_t *)q, ldq, s, lds);
    else
        hipLaunchKernelGGL(k_quant_act<_Float16>, dim3(grid_for(thr)), dim3(256), 0, (hipStream_t)stream,
                           (const _Float16 *)x, ldx, M, K, (uint8_t *)q, ldq, s, lds);
    return xt_check("eva_k_quant_act");
}

extern "C" int eva_k_quant_w(const float *w, int N, int K, void *q, float *s, void *stream)
{
    if (N <= 0 || K <= 0 || K % 128) return xt_fail("eva_k_quant_w", "bad shape (N > 0, K % 128 == 0)");
    if (((uintptr_t)w | (uintptr_t)q) & 15) return xt_fail("eva_k_quant_w", "w and q must be 16-byte aligned");
    hipLaunchKernelGGL(k_quant_w, dim3(K / 128, (N + 127) / 128), dim3(256), 0, (hipStream_t)stream, w, N, K,
                       (uint8_t *)q, s);
    return xt_check("eva_k_quant_w");
}

extern "C" int eva_k_e4m3_bits(uint32_t first, uint32_t count, void *out, void *stream)
{
    if (!count) return 0;
    hipLaunchKernelGGL(k_e4m3_bits, dim3(grid_for(count)), dim3(256), 0, (hipStream_t)stream, first, count,
                       (uint8_t *)out);
    return xt_check("eva_k_e4m3_bits");
}

extern "C" int eva_k_scale_bits(uint32_t first, uint32_t count, int which, void *out, void *stream)
{
    if (which != 0 && which != 1) return xt_fail("eva_k_scale_bits", "which must be 0 (scale) or 1 (inverse)");
    if (!count) return 0;
    hipLaunchKernelGGL(k_scale_bits, dim3(grid_for(count)), dim3(256), 0, (hipStream_t)stream, first, count, which,
                       (uint32_t *)out);
    return xt_check("eva_k_scale_bits");
}

template <bool SP>
static int gemm_launch(const char *what, const void *qa, int lda, const float *sa, int lds, const void *qw,
                       const void *qx, const float *sw, int M, int N, int K, void *c, int ldc, int out_kind,
                       void *stream)
{
    if (M < 0 || N <= 0 || K <= 0 || K % 128 || lda < K || lda % 16 || lds < M || ldc < N ||
        (out_kind != 0 && out_kind != 1))
        return xt_fail(what, "bad shape (K % 128, lda >= K and a multiple of 16, lds >= M, ldc >= N, out_kind 0 or 1)");
    if (((uintptr_t)qa | (uintptr_t)qw) & 15) return xt_fail(what, "qa and qw must be 16-byte aligned");
    // buffer descriptors and row offsets are 32-bit: operands and output must stay below 2 GiB (the A-row sentinel
    // XT_OOR = 2^31 must lie past every valid offset) and 4 GiB
    const size_t Np = ((size_t)N + 255) / 256 * 256;
    if ((size_t)M * lda >= (1u << 31) || Np * K >= (1u << 31) || (size_t)M * ldc * (out_kind ? 4 : 2) >= (1ull << 32) ||
        (size_t)lds * (K / 128) * 4 >= (1u << 31))
        return xt_fail(what, "operands too large for 32-bit offsets (M * lda, N * K < 2^31 bytes, C < 4 GiB)");
    if (SP && (N % 16 || !qx || ((uintptr_t)qx & 3))) return xt_fail(what, "sparse weights: N % 16 == 0, 4-byte aligned indices");
    if (!M) return 0;
    const uint8_t *A = (const uint8_t *)qa, *W = (const uint8_t *)qw;
    const uint32_t *X = (const uint32_t *)qx;
    hipStream_t st = (hipStream_t)stream;
    // big tiles once there are enough of them to fill the 256 CUs, else 128 x 128 tiles (two blocks per CU)
    const long big = (long)((M + GemmBig::BM - 1) / GemmBig::BM) * ((N + GemmBig::BN - 1) / GemmBig::BN);
    if (big >= 256) {
        const dim3 grid((unsigned)big);
        if (out_kind == 0)
            hipLaunchKernelGGL((k_gemm<GemmBig, 0, SP>), grid, dim3(GemmBig::NT), 0, st, A, lda, sa, lds, W, X, sw, c,
                               ldc, M, N, K);
        else
            hipLaunchKernelGGL((k_gemm<GemmBig, 1, SP>), grid, dim3(GemmBig::NT), 0, st, A, lda, sa, lds, W, X, sw, c,
                               ldc, M, N, K);
    } else {
        const dim3 grid((unsigned)(((M + GemmMid::BM - 1) / GemmMid::BM) * ((N + GemmMid::BN - 1) / GemmMid::BN)));
        if (out_kind == 0)
            hipLaunchKernelGGL((k_gemm<GemmMid, 0, SP>), grid, dim3(GemmMid::NT), 0, st, A, lda, sa, lds, W, X, sw, c,
                               ldc, M, N, K);
        else
            hipLaunchKernelGGL((k_gemm<GemmMid, 1, SP>), grid, dim3(GemmMid::NT), 0, st, A, lda, sa, lds, W, X, sw, c,
                               ldc, M, N, K);
    }
    return xt_check(what);
}

extern "C" int eva_k_gemm(const void *qa, int lda, const float *sa, int lds, const void *qw, const float *sw, int M,
                          int N, int K, void *c, int ldc, int out_kind, void *stream)
{
    return gemm_launch<false>("eva_k_gemm", qa, lda, sa, lds, qw, nullptr, sw, M, N, K, c, ldc, out_kind, stream);
}

extern "C" int eva_k_gemm_sp(const void *qa, int lda, const float *sa, int lds, const void *vals, const void *idx,
                             const float *sw, int M, int N, int K, void *c, int ldc, int out_kind, void *stream)
{
    return gemm_launch<true>("eva_k_gemm_sp", qa, lda, sa, lds, vals, idx, sw, M, N, K, c, ldc, out_kind, stream);
}
