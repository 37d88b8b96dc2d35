// gemm_core.h - block-scaled E4M3 GEMM main loop for gfx950 (the role of the reference's gemm8,
// src/engine/kern_common.cuh:271-356, generalised from one per-tensor alpha to per-block scales).
//
//   acc[m][n] = sum_kb sa[kb][m] * sw[n / 128][kb] * sum_{k in kb} A[m][k] * W[n][k]
//
// A [M][lda] E4M3 bytes (activations, 1x128 scales sa [K/128][lds]), W [Npad][K] E4M3 bytes (weights, 128x128
// scales sw [Npad/128][K/128], rows padded with zeros to a multiple of 128). K % 128 == 0.
//
// CDNA4 mapping:
//  - one K step = one 128-wide scale block = one v_mfma_f32_16x16x128_f8f6f4 per 16x16 output tile, so the block
//    partial leaves the matrix core whole and is promoted with one fma per accumulator: acc = fma(p, sa*sw, acc);
//  - operands go HBM/L2 -> LDS by buffer_load_dwordx4 ... lds (no VGPR staging): each wave instruction fills 1 KB
//    of LDS = 8 rows of 128 bytes; the XOR swizzle (16-byte chunk c of row r at chunk c ^ (r & 7)) is applied on the
//    global side by choosing which chunk each lane fetches. Buffer descriptors bound A and W, so rows past M (or past
//    the padded N) read as zero without a branch;
//  - two LDS stages, one barrier per K step; the next step's loads are in flight during this step's MFMAs;
//  - waves are laid out NWM x NWN, each owning a WM x WN sub-tile (WN inside one 128-column weight block). A wave
//    holds its TM A fragments and streams its TN B fragments.
#pragma once
#include "xt_common.h"

typedef __attribute__((address_space(3))) void lds_void;

#ifndef XT_LAG
#define XT_LAG 2      // MFMA -> promotion distance of the main-loop software pipeline
#endif
#ifndef XT_SGB
#define XT_SGB 1      // interleave hints (sched_group_barrier) in the main loop
#endif
#ifndef XT_GM
#define XT_GM 8       // grouped raster: row tiles walked together
#endif

template <int BM_, int BN_, int NWM_, int NWN_, int NS_ = 2>
struct BsCfg {
    static constexpr int BM = BM_, BN = BN_, NWM = NWM_, NWN = NWN_, NS = NS_;
    static constexpr int NW = NWM * NWN;
    static constexpr int NT = NW * 64;
    static constexpr int WM = BM / NWM, WN = BN / NWN;
    static constexpr int TM = WM / 16, TN = WN / 16;
    static constexpr int A_BYTES = BM * 128;
    static constexpr int B_BYTES = BN * 128;
    static constexpr int S_BYTES = BM * 4;
    static constexpr int STAGE = A_BYTES + B_BYTES + S_BYTES;
    static constexpr int LDS = NS * STAGE;
    static constexpr int LA = BM / (8 * NW);  // 1 KB A loads per wave per stage
    static constexpr int LB = BN / (8 * NW);  // 1 KB B loads per wave per stage
    static constexpr int LPS = LA + LB + 1;   // buffer loads per wave per stage (every wave loads one scale chunk)
    static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile must be whole 16x16 MFMA tiles");
    static_assert(WN <= 128 && 128 % WN == 0, "a wave's columns must sit in one weight block");
    static_assert(LA * 8 * NW == BM && LB * 8 * NW == BN, "tile rows must split evenly over the waves");
    static_assert(BM % 64 == 0 && BM / 64 <= NW, "one 256-byte scale load per wave");
    static_assert(NS >= 2 && LDS <= 160 * 1024, "the stages must fit the 160 KB LDS");
};

__device__ __forceinline__ uint32_t swz(int row, int chunk) { return (uint32_t)(row * 128 + ((chunk ^ (row & 7)) << 4)); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

// 16 bytes per lane from rsrc + voff into LDS at lds + 16 * lane (lds wave-uniform)
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, uint8_t *lds, uint32_t voff)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 16, (int)voff, 0, 0, 0);
}
__device__ __forceinline__ void lds_load4(__amdgpu_buffer_rsrc_t r, uint8_t *lds, uint32_t voff)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 4, (int)voff, 0, 0, 0);
}

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
template <int N>
__device__ __forceinline__ void wait_vmem_n()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// 32 bytes of swizzled LDS row `row` for lane group g (logical chunks 2g, 2g+1) as an MFMA operand. A and B use
// the same (lane group, byte) -> k map, so the product sums every k of the block exactly once.
__device__ __forceinline__ v8i ld_frag(const uint8_t *tile, int row, int g)
{
    const uint4 lo = *(const uint4 *)(tile + swz(row, 2 * g));
    const uint4 hi = *(const uint4 *)(tile + swz(row, 2 * g + 1));
    v8i v;
    v[0] = (int)lo.x; v[1] = (int)lo.y; v[2] = (int)lo.z; v[3] = (int)lo.w;
    v[4] = (int)hi.x; v[5] = (int)hi.y; v[6] = (int)hi.z; v[7] = (int)hi.w;
    return v;
}

template <class C>
struct BsOperands {
    // Per-lane parts of the load offsets live in one VGPR per operand; the wave-uniform parts (segment rows, K step)
    // go in the SGPR soffset of each buffer load.
    __amdgpu_buffer_rsrc_t ra, rw, rs;
    uint32_t a_lane, w_lane, s_lane;
    uint32_t a_seg, w_seg, s_plane;  // uniform: bytes between this wave's 8-row segments, scale plane bytes

    __device__ __forceinline__ void init(const uint8_t *A, int lda, const float *sa, int lds, const uint8_t *W,
                                         int K, int M, int Npad, int m0, int n0)
    {
        ra = buf_rsrc(A, (uint32_t)M * (uint32_t)lda);
        rw = buf_rsrc(W, (uint32_t)Npad * (uint32_t)K);
        rs = buf_rsrc(sa, (uint32_t)(K >> 7) * (uint32_t)lds * 4u);
        const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
        const int r8 = lane >> 3, c = (lane & 7) ^ r8;  // every segment starts on a multiple of 8 rows
        a_lane = (uint32_t)(m0 + 8 * w * C::LA + r8) * lda + c * 16;
        w_lane = (uint32_t)(n0 + 8 * w * C::LB + r8) * K + c * 16;
        s_lane = (uint32_t)(m0 + 64 * (w % (C::BM / 64)) + lane) * 4u;
        a_seg = 8u * lda;
        w_seg = 8u * K;
        s_plane = (uint32_t)lds * 4u;
    }

    __device__ __forceinline__ void issue(uint8_t *stage, int kb) const
    {
        const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
        for (int i = 0; i < C::LA; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void *)(stage + 1024 * (w * C::LA + i)), 16, (int)a_lane,
                                                     (int)(i * a_seg + kb * 128), 0, 0);
#pragma unroll
        for (int i = 0; i < C::LB; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_void *)(stage + C::A_BYTES + 1024 * (w * C::LB + i)), 16,
                                                     (int)w_lane, (int)(i * w_seg + kb * 128), 0, 0);
        // waves past BM / 64 repeat a scale chunk (same bytes to the same place) so every wave issues LPS loads
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void *)(stage + C::A_BYTES + C::B_BYTES + 256 * (w % (C::BM / 64))),
                                                 4, (int)s_lane, (int)(kb * s_plane), 0, 0);
    }
};

template <class C>
__device__ __forceinline__ void bs_wave_origin(int &wm0, int &wn0)
{
    const int w = threadIdx.x >> 6;
    wm0 = (w / C::NWN) * C::WM;
    wn0 = (w % C::NWN) * C::WN;
}

// Main loop. On return acc[i][j][r] holds output row m0 + wm0 + 16 i + 4 (lane >> 4) + r, column
// n0 + wn0 + 16 j + (lane & 15), where (wm0, wn0) = bs_wave_origin(). The block is synchronised and the whole
// shared memory is free for the epilogue.
template <class C>
__device__ __forceinline__ void bs_mainloop(const uint8_t *__restrict__ A, int lda, const float *__restrict__ sa,
                                            int lds, const uint8_t *__restrict__ W, const float *__restrict__ sw,
                                            int M, int Npad, int K, int m0, int n0, uint8_t *smem,
                                            v4f (&acc)[C::TM][C::TN])
{
    BsOperands<C> op;
    const int lane = threadIdx.x & 63, g = lane >> 4, r16 = lane & 15;
    const int KB = K >> 7;
    int wm0, wn0;
    bs_wave_origin<C>(wm0, wn0);
    const float *swp = sw + (size_t)__builtin_amdgcn_readfirstlane((n0 + wn0) >> 7) * KB;
    op.init(A, lda, sa, lds, W, K, M, Npad, m0, n0);

#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int j = 0; j < C::TN; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int s = 0; s < C::NS - 1; s++)
        if (s < KB) op.issue(smem + s * C::STAGE, s);
    if (KB >= C::NS - 1) wait_vmem_n<(C::NS - 2) * C::LPS>();
    else wait_vmem();
    __syncthreads();
    int cs = 0, is = C::NS - 1;  // stage computed now, stage issued now
    for (int kb = 0; kb < KB; kb++) {
        const uint8_t *st = smem + cs * C::STAGE;
        const bool more = kb + C::NS - 1 < KB;
        if (more) op.issue(smem + is * C::STAGE, kb + C::NS - 1);
        const float swv = swp[kb];  // wave-uniform pointer: a scalar load, off the vector-memory counter
        const uint8_t *ta = st, *tb = st + C::A_BYTES;
        const float *ts = (const float *)(st + C::A_BYTES + C::B_BYTES);
        v8i a[C::TM];
        v4f sc[C::TM];
#pragma unroll
        for (int i = 0; i < C::TM; i++) {
            a[i] = ld_frag(ta, wm0 + 16 * i + r16, g);
            const float4 s4 = *(const float4 *)(ts + wm0 + 16 * i + 4 * g);
            sc[i] = v4f{s4.x * swv, s4.y * swv, s4.z * swv, s4.w * swv};
        }
        // Software pipeline over the TN x TM MFMAs of this K step: MFMA number t is issued, then the four
        // promotion fmas of MFMA t - 2, whose result has had two MFMA slots to land. One wave thus keeps the matrix
        // core busy while its VALU promotes; B fragments are read one column tile ahead.
        constexpr int NS = C::TN * C::TM, LAG = XT_LAG;
        v4f pr[LAG + 1];
        v8i bcur = ld_frag(tb, wn0 + r16, g), bnext = bcur;
#pragma unroll
        for (int t = 0; t < NS + LAG; t++) {
            if (t < NS) {
                const int j = t / C::TM, i = t % C::TM;
                if (i == 0 && j + 1 < C::TN) bnext = ld_frag(tb, wn0 + 16 * (j + 1) + r16, g);
                pr[t % (LAG + 1)] = mfma_e4m3_16x16x128(a[i], bcur);
                if (i == C::TM - 1) bcur = bnext;
                if (XT_SGB) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
            }
            if (t >= LAG) {
                const int u = t - LAG, j = u / C::TM, i = u % C::TM;
                const v4f p = pr[u % (LAG + 1)];
                acc[i][j][0] = __builtin_fmaf(p[0], sc[i][0], acc[i][j][0]);
                acc[i][j][1] = __builtin_fmaf(p[1], sc[i][1], acc[i][j][1]);
                acc[i][j][2] = __builtin_fmaf(p[2], sc[i][2], acc[i][j][2]);
                acc[i][j][3] = __builtin_fmaf(p[3], sc[i][3], acc[i][j][3]);
                if (XT_SGB) __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // then 4 VALU
            }
        }
        // stage kb + 1 must be resident: the NS - 2 stages issued after it may stay in flight
        if (more) wait_vmem_n<(C::NS - 2) * C::LPS>();
        else wait_vmem();
        __syncthreads();
        cs = cs == C::NS - 1 ? 0 : cs + 1;
        is = is == C::NS - 1 ? 0 : is + 1;
    }
}

// XCD-aware tile order for a 1-D grid of T = tiles_m * tiles_n blocks. Blocks are dispatched to the 8 XCDs round
// robin (block b -> XCD b % 8), so XCD x is given a contiguous run of a grouped raster (XT_GM row tiles walked
// together across all column tiles): the ~32 blocks an XCD runs at once share a few A row tiles and W column tiles
// in that XCD's L2.
__device__ __forceinline__ void tile_of_block(int tiles_m, int tiles_n, int &tm, int &tn)
{
    const int T = tiles_m * tiles_n, b = blockIdx.x, x = b & 7, q = T >> 3, r = T & 7;
    const int pos = x * q + (x < r ? x : r) + (b >> 3);
    const int per_group = XT_GM * tiles_n, grp = pos / per_group, rem = pos - grp * per_group;
    const int gm = tiles_m - grp * XT_GM < XT_GM ? tiles_m - grp * XT_GM : XT_GM;
    tm = grp * XT_GM + rem % gm;
    tn = rem / gm;
}
