// layer_core.h - pieces shared by the block-GEMM kernels of the EVA02-L (wd) and ViTDet-L (PixAI) layers: the tile
// configuration, the shared-memory plan of the epilogues, the main-loop dispatch (dense or 2:4-sparse weights), the
// tile raster and the residual update of a wave tile.
#pragma once
#include "gemm_core.h"
#include "xt_abi.h"

typedef BsCfg<256, 256, 4, 2, 2> LayerCfg;  // 8 waves of 64 x 128: two heads (qkv) or 64 SwiGLU units (fc1) per wave

// Shared memory of the layer kernels: the main-loop stages, reused by the epilogues (one 64 x 68 fp32 residual slice
// per wave, one [128][68] bf16 transpose slice per wave, or the fc1 h tile), then 2 KB of per-row statistics and
// 2 KB of per-column fold terms that k_fc2 fills while its first stages load.
constexpr int LAYER_RES_SLICE = 64 * 68 * 4;
constexpr int LAYER_ROWSTAT = LayerCfg::NW * LAYER_RES_SLICE;  // byte offset of the per-row statistics
constexpr int LAYER_SMEM = LAYER_ROWSTAT + 4096;                 // 2 KB row statistics + 2 KB column terms
static_assert(LAYER_ROWSTAT >= LayerCfg::LDS, "row statistics sit past the main-loop stages");
static_assert(LAYER_SMEM <= 160 * 1024, "layer kernels fit the LDS");
static_assert(LayerCfg::NW * 128 * 68 * 2 <= LAYER_ROWSTAT, "v transpose slices fit");

__device__ __forceinline__ uint32_t pk_bf16(float a, float b)
{
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{a, b}), b2));
}

// two fp32 values rounded to fp16 (RNE) in one v_cvt_pk_f16_f32, a in the low half
__device__ __forceinline__ uint32_t pk_f16(float a, float b)
{
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    asm volatile("" : "+v"(a), "+v"(b));  // fp32 values: no fused fp32-op + fp16-round (v_fma_mix*) single rounding
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{a, b}), h2));
}

// The layer kernels take their weights dense (w, wx unused) or 2:4-sparse (SP: w = pack24 values, wx = indices).
// Nlive (default Npad): columns from Nlive on hold zero weights throughout, so waves that own only such columns skip
// their matrix work.
// TR (dense weights only): the tile transposed, as bs_mainloop's TR leaves it.
template <class C, bool SP, class Pre = BsNoPre, bool TR = false>
__device__ __forceinline__ void layer_mainloop(const uint8_t *A, int lda, const float *sa, int lds, const uint8_t *w,
                                               const uint32_t *wx, const float *ws, int rows, int Npad, int K, int m0,
                                               int n0, uint8_t *smem, v4f (&acc)[C::TM][C::TN], Pre pre = Pre(),
                                               int Nlive = -1)
{
    static_assert(!SP || C::LDS_SP <= LAYER_ROWSTAT, "sparse stages end before the row statistics");
    static_assert(!(SP && TR), "the sparse tile comes transposed from bs_mainloop_sp_t");
    if constexpr (SP) bs_mainloop_sp<C>(A, lda, sa, lds, w, wx, ws, rows, Npad, K, m0, n0, smem, acc, pre, Nlive);
    else bs_mainloop<C, Pre, true, TR>(A, lda, sa, lds, w, ws, rows, Npad, K, m0, n0, smem, acc, pre, Nlive);
}

template <class C>
__device__ __forceinline__ void layer_tile(int M, int N, int &m0, int &n0)
{
    int tm, tn;
    tile_of_block((M + C::BM - 1) / C::BM, (N + C::BN - 1) / C::BN, M % C::BM != 0, tm, tn);
    m0 = tm * C::BM;
    n0 = tn * C::BN;
}

// Residual update x = f16(x + y) of a wave's 64 x (16 TN) tile, y in the MFMA C layout, in passes of 64 columns.
// The wave parks 64 x 64 of y in its own LDS slice (row stride 68 floats: the 64 lanes of one store hit 64 different
// banks), then each lane updates 8 consecutive halves with one 16-byte load and store, so one wave instruction
// covers 8 rows of 128 bytes. Every x load of the tile is issued before the first store (one memory round trip for
// the whole update), through a buffer descriptor that ends at row `rows`: rows past it load zero and their stores
// are dropped, with no branch between the loads.
struct ResIdentity {
    __device__ __forceinline__ float operator()(int, int, int, float v) const { return v; }
};

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// x + y for the fp16 x in the low (HI = 0) or high (HI = 1) half of a word and an fp32 y: one v_fma_mix_f32,
// fma(x, 1, y) with x widened exactly, which rounds once to fp32 as the conversion followed by v_add_f32 does
template <int HI>
__device__ __forceinline__ float h_add(uint32_t xw, float y)
{
    float r;
    if constexpr (HI) asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(xw), "v"(y));
    else asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[0,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(xw), "v"(y));
    return r;
}

// f(i, j, r, y) maps each accumulator to the value added (row m0 + mw + 16 i + 4 (lane >> 4) + r, column tile j).
template <class C, class F = ResIdentity>
__device__ __forceinline__ void residual_add(uint8_t *slices, v4f (&y)[C::TM][C::TN], uint16_t *__restrict__ x,
                                             int mw, int nw, int rows, F f = F())
{
    static_assert(C::TM == 4 && C::TN % 4 == 0, "64-row wave tiles, whole 64-column passes");
    constexpr int NP = C::TN / 4;
    float *tr = (float *)(slices + (threadIdx.x >> 6) * LAYER_RES_SLICE);
    const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    const int rs = lane >> 3, ch = lane & 7;
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, (uint32_t)rows * XT_D * 2u);
    const uint32_t off0 = (uint32_t)(((mw + rs) * XT_D + nw + 8 * ch) * 2);
    v4u xv[NP][8];
#pragma unroll
    for (int pass = 0; pass < NP; pass++)
#pragma unroll
        for (int it = 0; it < 8; it++)
            xv[pass][it] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(off0 + (uint32_t)((8 * it * XT_D + 64 * pass) * 2)), 0, 0);
#pragma unroll
    for (int pass = 0; pass < NP; pass++) {
        if (pass) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the previous pass's slice reads are done
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    tr[(16 * i + 4 * g + r) * 68 + 16 * j + c16] = f(i, 4 * pass + j, r, y[i][4 * pass + j][r]);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slice is the wave's own: no block barrier needed
#pragma unroll
        for (int it = 0; it < 8; it++) {
            const int rr = 8 * it + rs;
            const float4 a = *(const float4 *)(tr + rr * 68 + 8 * ch), b = *(const float4 *)(tr + rr * 68 + 8 * ch + 4);
            const v4u v = xv[pass][it];
            v4u o;
            o[0] = pk_f16(h_add<0>(v[0], a.x), h_add<1>(v[0], a.y));
            o[1] = pk_f16(h_add<0>(v[1], a.z), h_add<1>(v[1], a.w));
            o[2] = pk_f16(h_add<0>(v[2], b.x), h_add<1>(v[2], b.y));
            o[3] = pk_f16(h_add<0>(v[3], b.z), h_add<1>(v[3], b.w));
            __builtin_amdgcn_raw_buffer_store_b128(o, rx, (int)(off0 + (uint32_t)((8 * it * XT_D + 64 * pass) * 2)), 0, 0);
        }
    }
}

// residual_add for a transposed tile (the sparse main loop's, or bs_mainloop's with TR): y(jn, im) gives the four
// values added to row mw + 16 im + (lane & 15), columns nw + 16 jn + 4 (lane >> 4) + r. The same update, with the
// tile parked in the slice by one 16-byte store per (m tile, n tile) (row stride 68 floats: the 16 rows of one store
// group start 4 banks apart).
template <class C, class Y>
__device__ __forceinline__ void residual_add_t(uint8_t *slices, Y y, uint16_t *__restrict__ x, int mw, int nw, int rows)
{
    static_assert(C::TM == 4 && C::TN % 4 == 0, "64-row wave tiles, whole 64-column passes");
    constexpr int NP = C::TN / 4;
    float *tr = (float *)(slices + (threadIdx.x >> 6) * LAYER_RES_SLICE);
    const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    const int rs = lane >> 3, ch = lane & 7;
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, (uint32_t)rows * XT_D * 2u);
    const uint32_t off0 = (uint32_t)(((mw + rs) * XT_D + nw + 8 * ch) * 2);
    v4u xv[NP][8];
#pragma unroll
    for (int pass = 0; pass < NP; pass++)
#pragma unroll
        for (int it = 0; it < 8; it++)
            xv[pass][it] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(off0 + (uint32_t)((8 * it * XT_D + 64 * pass) * 2)), 0, 0);
#pragma unroll
    for (int pass = 0; pass < NP; pass++) {
        if (pass) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the previous pass's slice reads are done
#pragma unroll
        for (int im = 0; im < 4; im++)
#pragma unroll
            for (int jq = 0; jq < 4; jq++) {
                const v4f v = y(4 * pass + jq, im);
                *(float4 *)(tr + (16 * im + c16) * 68 + 16 * jq + 4 * g) = make_float4(v[0], v[1], v[2], v[3]);
            }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slice is the wave's own: no block barrier needed
#pragma unroll
        for (int it = 0; it < 8; it++) {
            const int rr = 8 * it + rs;
            const float4 a = *(const float4 *)(tr + rr * 68 + 8 * ch), b = *(const float4 *)(tr + rr * 68 + 8 * ch + 4);
            const v4u v = xv[pass][it];
            v4u o;
            o[0] = pk_f16(h_add<0>(v[0], a.x), h_add<1>(v[0], a.y));
            o[1] = pk_f16(h_add<0>(v[1], a.z), h_add<1>(v[1], a.w));
            o[2] = pk_f16(h_add<0>(v[2], b.x), h_add<1>(v[2], b.y));
            o[3] = pk_f16(h_add<0>(v[3], b.z), h_add<1>(v[3], b.w));
            __builtin_amdgcn_raw_buffer_store_b128(o, rx, (int)(off0 + (uint32_t)((8 * it * XT_D + 64 * pass) * 2)), 0, 0);
        }
    }
}

static inline unsigned layer_grid(int rows, int N, int BM, int BN)
{
    return (unsigned)(((rows + BM - 1) / BM) * ((N + BN - 1) / BN));
}

#define XT_ALIGNED(p) ((((uintptr_t)(p)) & 15) == 0)

// Token rows a layer launcher accepts: every 32-bit buffer offset (rows x 4736 bytes of the widest E4M3 activation,
// rows x 2048 of an fp16 residual or bf16 q / k, the XT_OOR = 2^31 sentinel of rows past the end) stays in range.
static inline int layer_rows_ok(const char *what, int rows, int lds)
{
    if (rows <= 0 || lds < rows || rows > (1 << 19)) return xt_fail(what, "bad shape (0 < rows <= 2^19, lds >= rows)");
    return 0;
}
