// gemm_core.h - block-scaled E4M3 GEMM main loop for gfx950 (the role of the reference's gemm8,
// src/engine/kern_common.cuh:271-356, generalised from one per-tensor alpha to per-block scales).
//
//   acc[m][n] = sum_kb sa[kb][m] * sw[n / 128][kb] * sum_{k in kb} A[m][k] * W[n][k]
//
// A [M][lda] E4M3 bytes (activations, 1x128 scales sa [K/128][lds]), W [Npad][K] E4M3 bytes (weights, 128x128
// scales sw [Npad/128][K/128], rows padded with zeros to a multiple of 128). K % 128 == 0.
//
// CDNA4 mapping:
//  - one K step = one 128-wide scale block = one MFMA per 16x16 output tile: the block partial leaves the matrix core
//    whole (v_mfma_f32_16x16x128_f8f6f4, fp32 result) and is promoted with one fma per accumulator,
//    acc = fma(p, sa * sw, acc), so any fp32 scales are honoured (the reference's alpha * acc, eva.h:415-418, with the
//    scale product taken per row and per K block);
//  - operands go HBM/L2 -> LDS by buffer_load_dwordx4 ... lds (no VGPR staging), 1 KB = 8 rows x 128 bytes (whole
//    cache lines) per wave instruction. The loads are issued from inline assembly: the compiler then does not track
//    them, and its conservative "wait for every LDS DMA before any LDS read" rule (which would drain the whole
//    prefetch pipeline every K step) is replaced by exact vmcnt waits below;
//  - LDS tiles are row-major, 128 bytes per row, with 16-byte chunk c of row r rotated to chunk (c + r) & 7. Lane
//    (g, r) of an operand fragment holds chunks g and g + 4 of its row; both ds_read_b128 of a fragment then run at
//    the full LDS rate on gfx950 (measured: an XOR swizzle of the same reads runs at half of it). The rotation is
//    applied on the global side, by choosing which chunk of its row each DMA lane fetches;
//  - every row offset is in the per-lane VGPR offset and only the K step in the SGPR offset, so rows past M (or past
//    the padded N) fail the buffer range check and load as zero whether or not the SGPR offset is range-checked;
//  - NS LDS stages, one barrier per K step; the next NS - 1 steps' loads are in flight during this step's MFMAs;
//  - waves are laid out NWM x NWN, each owning a WM x WN sub-tile (WN inside one 128-column weight block). A wave
//    holds its TM A fragments and streams its TN B fragments one column tile ahead.
#pragma once
#include "xt_common.h"

typedef __attribute__((address_space(3))) void lds_void;
typedef int v4i __attribute__((ext_vector_type(4)));

#ifndef XT_LAG
#define XT_LAG 2      // MFMA -> promotion distance of the main-loop software pipeline
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
    static constexpr int S_BYTES = BM * 4;     // activation scales of the BM rows
    static constexpr int SW_BYTES = 256;       // weight scales of the BN / 128 column blocks (one 64-lane dword load)
    static constexpr int STAGE = A_BYTES + B_BYTES + S_BYTES + SW_BYTES;
    static constexpr int LDS = NS * STAGE;
    static constexpr int LA = BM / (8 * NW);  // 1 KB A loads (8 rows) per wave per stage
    static constexpr int LB = BN / (8 * NW);  // 1 KB B loads per wave per stage
    static constexpr int SL = BM / 64;        // 256-byte activation-scale loads per stage (waves 0 .. SL-1)
    static constexpr int LPS = LA + LB + 1;   // loads per wave per stage: every wave issues one dword load
    static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile must be whole 16x16 MFMA tiles");
    static_assert(WN <= 128 && 128 % WN == 0, "a wave's columns must sit in one weight block");
    static_assert(LA * 8 * NW == BM && LB * 8 * NW == BN, "tile rows must split evenly over the waves");
    static_assert(BM % 64 == 0 && SL < NW, "scale loads: one wave per 64 rows plus one for the weight scales");
    static_assert(BN / 128 <= 64, "weight-scale load covers at most 64 column blocks");
    static_assert(NS >= 2 && LDS <= 160 * 1024, "the stages must fit the 160 KB LDS");
    // 2:4-sparse weights (bs_mainloop_sp): per stage BN / 16 compressed 1 KB value blocks and 256-byte index blocks
    static constexpr int LV = BN / (16 * NW);   // value (and index) blocks per wave per stage
    static constexpr int V_BYTES = BN * 64;
    static constexpr int X_BYTES = BN * 16;
    static constexpr int STAGE_SP = A_BYTES + V_BYTES + X_BYTES + S_BYTES + SW_BYTES;
    static constexpr int LDS_SP = NS * STAGE_SP + 16;  // the stages, then the 16 zero bytes of bs_step_sp
    static constexpr int LPS_SP = LA + 2 * LV + 1;
};

// 16-byte chunk swizzle of the attention and patch-embedding tiles (chunk c of row r at c ^ (r & 7))
__device__ __forceinline__ uint32_t swz(int row, int chunk) { return (uint32_t)(row * 128 + ((chunk ^ (row & 7)) << 4)); }

// Raw buffer descriptor (base, stride 0, num_records = bytes, 32-bit dword format) in SGPRs.
__device__ __forceinline__ v4i buf_desc(const void *p, uint32_t bytes)
{
    const uint64_t a = (uint64_t)(uintptr_t)p;
    v4i r;
    r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
    r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
    r[3] = 0x00020000;
    return r;
}

// LDS address (byte offset in the workgroup's LDS) of a shared-memory pointer
__device__ __forceinline__ uint32_t lds_addr(const void *p) { return (uint32_t)(uintptr_t)(lds_void *)p; }

// buffer_load ... lds: lane l's 16 (4) bytes from rsrc + voff + soff land at LDS m0 + 16 l (4 l). m0 and soff are
// wave-uniform. Not visible to the compiler's wait-count tracking: callers wait with wait_vmem*.
__device__ __forceinline__ void dma16(v4i r, uint32_t m0, uint32_t voff, uint32_t soff)
{
    asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(m0), "v"(voff), "s"(r), "s"(soff) : "memory");
}
__device__ __forceinline__ void dma4(v4i r, uint32_t m0, uint32_t voff, uint32_t soff)
{
    asm volatile("buffer_load_dword %1, %2, %3 offen lds" ::"{m0}"(m0), "v"(voff), "s"(r), "s"(soff) : "memory");
}

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
template <int N>
__device__ __forceinline__ void wait_vmem_n()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// block barrier after this wave's LDS reads have returned; no fence (the LDS DMA waits are explicit)
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// MFMA operand fragment of the 16-row tile starting at tile row r0 (a multiple of 16): lane (g, r) gets chunks g
// and g + 4 of row r0 + r. A and B use the same (lane group, byte) -> k map, so the product sums every k of the
// 128-wide block exactly once.
__device__ __forceinline__ v8i ld_frag(const uint8_t *tile, int r0)
{
    const int lane = threadIdx.x & 63, g = lane >> 4, r = lane & 15;
    const uint8_t *p = tile + (r0 + r) * 128;
    const uint4 lo = *(const uint4 *)(p + (((g + r) & 7) << 4));
    const uint4 hi = *(const uint4 *)(p + (((g + 4 + r) & 7) << 4));
    v8i v;
    v[0] = (int)lo.x; v[1] = (int)lo.y; v[2] = (int)lo.z; v[3] = (int)lo.w;
    v[4] = (int)hi.x; v[5] = (int)hi.y; v[6] = (int)hi.z; v[7] = (int)hi.w;
    return v;
}

#define XT_OOR 0x80000000u  // a buffer offset past every range used here: the load returns zero

template <class C>
struct BsOperands {
    v4i ra, rw, rs;                 // A, W and the scale source of this wave's dword load (sa or sw)
    uint32_t a_off[C::LA], w_off[C::LB], s_off;
    uint32_t s_step;                // SGPR offset of one K step for the dword load (sa plane or one sw float)
    uint32_t m0_a, m0_b, m0_s;      // LDS byte offsets of this wave's slots inside a stage

    __device__ __forceinline__ void init(const uint8_t *A, int lda, const float *sa, int lds, const uint8_t *W,
                                         const float *sw, int K, int M, int Npad, int m0, int n0)
    {
        const int KB = K >> 7;
        ra = buf_desc(A, (uint32_t)M * (uint32_t)lda);
        rw = buf_desc(W, (uint32_t)Npad * (uint32_t)K);
        const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
        const int r8 = lane >> 3, p = lane & 7;
#pragma unroll
        for (int i = 0; i < C::LA; i++) {  // 1 KB block q = tile rows 8q .. 8q+7; lane slot p holds chunk (p - row) & 7
            const int rl = 8 * (w * C::LA + i) + r8, m = m0 + rl;
            a_off[i] = m < M ? (uint32_t)m * (uint32_t)lda + (uint32_t)(((p - rl) & 7) << 4) : XT_OOR;
        }
#pragma unroll
        for (int i = 0; i < C::LB; i++) {
            const int rl = 8 * (w * C::LB + i) + r8, n = n0 + rl;
            w_off[i] = n < Npad ? (uint32_t)n * (uint32_t)K + (uint32_t)(((p - rl) & 7) << 4) : XT_OOR;
        }
        m0_a = (uint32_t)(1024 * w * C::LA);
        m0_b = (uint32_t)(C::A_BYTES + 1024 * w * C::LB);
        if (w < C::SL) {            // activation scales of rows m0 + 64 w + lane, plane kb
            rs = buf_desc(sa, (uint32_t)KB * (uint32_t)lds * 4u);
            const int m = m0 + 64 * w + lane;
            s_off = m < lds ? (uint32_t)m * 4u : XT_OOR;
            s_step = (uint32_t)lds * 4u;
            m0_s = (uint32_t)(C::A_BYTES + C::B_BYTES + 256 * w);
        } else {                    // weight scales of column blocks n0 / 128 + lane (the last waves repeat it)
            const int nbt = Npad >> 7, nb = (n0 >> 7) + lane;
            rs = buf_desc(sw, (uint32_t)nbt * (uint32_t)KB * 4u);
            s_off = (lane < C::BN / 128 && nb < nbt) ? (uint32_t)(nb * KB) * 4u : XT_OOR;
            s_step = 4u;
            m0_s = (uint32_t)(C::A_BYTES + C::B_BYTES + C::S_BYTES);
        }
    }

    // all LPS loads of K step kb into the stage at LDS byte offset stage
    __device__ __forceinline__ void issue(uint32_t stage, int kb) const
    {
        const uint32_t koff = (uint32_t)kb * 128u;
#pragma unroll
        for (int i = 0; i < C::LA; i++) dma16(ra, stage + m0_a + 1024u * i, a_off[i], koff);
#pragma unroll
        for (int i = 0; i < C::LB; i++) dma16(rw, stage + m0_b + 1024u * i, w_off[i], koff);
        dma4(rs, stage + m0_s, s_off, (uint32_t)kb * s_step);
    }
    // load q (0 .. LPS - 1) of K step kb: the same loads as issue(), one at a time
    __device__ __forceinline__ void issue_one(int q, uint32_t stage, int kb) const
    {
        const uint32_t koff = (uint32_t)kb * 128u;
        if (q < C::LA) dma16(ra, stage + m0_a + 1024u * q, a_off[q], koff);
        else if (q < C::LA + C::LB) dma16(rw, stage + m0_b + 1024u * (q - C::LA), w_off[q - C::LA], koff);
        else dma4(rs, stage + m0_s, s_off, (uint32_t)kb * s_step);
    }
};

template <class C>
__device__ __forceinline__ void bs_wave_origin(int &wm0, int &wn0)
{
    const int w = threadIdx.x >> 6;
    wm0 = (w / C::NWN) * C::WM;
    wn0 = (w % C::NWN) * C::WN;
}

// One K step on a resident stage: TM x TN MFMAs, each block partial promoted into acc.
template <class C>
__device__ __forceinline__ void bs_step(const uint8_t *st, int wm0, int wn0, v4f (&acc)[C::TM][C::TN])
{
    const int lane = threadIdx.x & 63, g = lane >> 4;
    const uint8_t *ta = st, *tb = st + C::A_BYTES;
    const float *ts = (const float *)(st + C::A_BYTES + C::B_BYTES);
    const float swv = *(const float *)(st + C::A_BYTES + C::B_BYTES + C::S_BYTES + 4 * (wn0 >> 7));
    v8i a[C::TM];
    v4f sc[C::TM];
    v8i bcur = ld_frag(tb, wn0), bnext = bcur;
#pragma unroll
    for (int i = 0; i < C::TM; i++) a[i] = ld_frag(ta, wm0 + 16 * i);
#pragma unroll
    for (int i = 0; i < C::TM; i++) {
        const float4 s4 = *(const float4 *)(ts + wm0 + 16 * i + 4 * g);
        sc[i] = v4f{s4.x * swv, s4.y * swv, s4.z * swv, s4.w * swv};
    }
    // Software pipeline over the TN x TM MFMAs: MFMA number t is issued, then the four promotion fmas of MFMA
    // t - LAG, whose result has had LAG MFMA slots to land; B fragments are read one column tile ahead.
    constexpr int NS = C::TN * C::TM, LAG = XT_LAG;
    v4f pr[LAG + 1];
#pragma unroll
    for (int t = 0; t < NS + LAG; t++) {
        if (t < NS) {
            const int j = t / C::TM, i = t % C::TM;
            if (i == 0 && j + 1 < C::TN) bnext = ld_frag(tb, wn0 + 16 * (j + 1));
            pr[t % (LAG + 1)] = mfma_e4m3_16x16x128(a[i], bcur);
            if (i == C::TM - 1) bcur = bnext;
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        }
        if (t >= LAG) {
            const int u = t - LAG, j = u / C::TM, i = u % C::TM;
            const v4f p = pr[u % (LAG + 1)];
            acc[i][j][0] = __builtin_fmaf(p[0], sc[i][0], acc[i][j][0]);
            acc[i][j][1] = __builtin_fmaf(p[1], sc[i][1], acc[i][j][1]);
            acc[i][j][2] = __builtin_fmaf(p[2], sc[i][2], acc[i][j][2]);
            acc[i][j][3] = __builtin_fmaf(p[3], sc[i][3], acc[i][j][3]);
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // then 4 VALU
        }
    }
}

// The same K step for 64 x 128 and 64 x 64 wave tiles (TM = 4, TN = 8 or 4) in a fixed issue order (for 64 x 64, the
// single GEMM's 128 x 128 tiles, 12% faster than bs_step at M = 1025). The matrix-core instructions and
// the promotion fmas are single-instruction asm statements, and every LDS read sits between them, so the compiler
// keeps the written order (it still allocates registers and places the LDS waits):
//  - A 0 and B 0 are read first, then the scales, then A 1-3 and B 1: the first MFMA waits for four reads only;
//  - B fragment j + 2 is read right after MFMA (j, 0), into the slot B fragment j - 1 has left (3-slot ring);
//  - the promotion of MFMA t - 3 follows MFMA t (15 instructions separate an MFMA from the first VALU read of its
//    result; gfx950 asks 12 wait states); the promotion of MFMA 0 is preceded by s_nop 7. The step's last three
//    MFMAs are promoted at the start of the next step (pr and scp carry their results and scales), between the
//    first fragment reads and the first MFMA, where the wave would otherwise wait for the reads; the K loop
//    promotes the last step's three after it (bs_step_fixed_flush). Each accumulator still takes its K blocks in
//    order, so the sums are those of promoting at the end of each step, bit for bit;
//  - the LPS loads of K step dkb (dkb < 0: none) go out one per MFMA from MFMA 1 on, not in a burst that would stall
//    this wave's issue behind the vector-memory queue.
__device__ __forceinline__ void mfma_asm(v4f &p, const v8i &a, const v8i &b)
{
    asm volatile("v_mfma_f32_16x16x128_f8f6f4 %0, %1, %2, 0" : "=&v"(p) : "v"(a), "v"(b) : "memory");
}
__device__ __forceinline__ void fmac_asm(float &acc, float p, float s)
{
    asm volatile("v_fmac_f32 %0, %1, %2" : "+v"(acc) : "v"(p), "v"(s) : "memory");
}

// Promotion of a step's last three MFMAs (row tiles 1-3 of the last column tile, ring slots 1-3) with that step's
// scales scp
template <class C, bool TR = false>
__device__ __forceinline__ void bs_step_fixed_flush(v4f (&acc)[C::TM][C::TN], const v4f (&pr)[4],
                                                    const float (&scp)[3][4])
{
    constexpr int J = C::TN - 1;
#pragma unroll
    for (int q = 0; q < 3; q++) {
        const v4f p = pr[1 + q];
        float x0 = acc[1 + q][J][0], x1 = acc[1 + q][J][1], x2 = acc[1 + q][J][2], x3 = acc[1 + q][J][3];
        fmac_asm(x0, p[0], scp[q][0]);
        fmac_asm(x1, p[1], scp[q][TR ? 0 : 1]);
        fmac_asm(x2, p[2], scp[q][TR ? 0 : 2]);
        fmac_asm(x3, p[3], scp[q][TR ? 0 : 3]);
        acc[1 + q][J] = v4f{x0, x1, x2, x3};
    }
}

template <class C, bool TR = false>
__device__ __forceinline__ void bs_step_fixed(const uint8_t *st, int wm0, int wn0, v4f (&acc)[C::TM][C::TN],
                                              const BsOperands<C> &op, uint32_t dstage, int dkb, v4f (&pr)[4],
                                              float (&scp)[3][4], bool carry)
{
    static_assert(C::TM == 4 && (C::TN == 8 || C::TN == 4) && C::LPS < 4 * C::TN,
                  "schedule written for 64 x 128 and 64 x 64 wave tiles");
    constexpr int LAG = 3, NM = 4 * C::TN;
    const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    const uint8_t *ta = st, *tb = st + C::A_BYTES;
    const float *ts = (const float *)(st + C::A_BYTES + C::B_BYTES);
    v8i a[4], b[3];
    b[0] = ld_frag(tb, wn0);
    a[0] = ld_frag(ta, wm0);
    asm volatile("" ::: "memory");  // the first MFMA waits for these four reads only
    if (carry) bs_step_fixed_flush<C, TR>(acc, pr, scp);  // the previous step's last three MFMAs, while the reads land
    const float swv = *(const float *)(st + C::A_BYTES + C::B_BYTES + C::S_BYTES + 4 * (wn0 >> 7));
    float4 s4[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if constexpr (TR) s4[i].x = ts[wm0 + 16 * i + c16];  // TR: one row per lane and row tile
        else s4[i] = *(const float4 *)(ts + wm0 + 16 * i + 4 * g);
    }
    asm volatile("" ::: "memory");
    a[1] = ld_frag(ta, wm0 + 16);
    a[2] = ld_frag(ta, wm0 + 32);
    a[3] = ld_frag(ta, wm0 + 48);
    b[1] = ld_frag(tb, wn0 + 16);
    asm volatile("" ::: "memory");
    float sc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if constexpr (TR) {
            sc[i][0] = s4[i].x * swv;
        } else {
            sc[i][0] = s4[i].x * swv; sc[i][1] = s4[i].y * swv; sc[i][2] = s4[i].z * swv; sc[i][3] = s4[i].w * swv;
        }
    }
#pragma unroll
    for (int t = 0; t < NM; t++) {
        const int j = t >> 2, i = t & 3;
        if constexpr (TR) mfma_asm(pr[t % (LAG + 1)], b[j % 3], a[i]);  // the tile transposed: weights as A
        else mfma_asm(pr[t % (LAG + 1)], a[i], b[j % 3]);
        if (i == 0 && j + 2 < C::TN) b[(j + 2) % 3] = ld_frag(tb, wn0 + 16 * (j + 2));
        if (t >= 1 && t <= C::LPS && dkb >= 0) op.issue_one(t - 1, dstage, dkb);
        if (t == LAG) asm volatile("s_nop 7" ::: "memory");
        if (t >= LAG) {
            const int u = t - LAG, ju = u >> 2, iu = u & 3;
            const v4f p = pr[u % (LAG + 1)];
            float x0 = acc[iu][ju][0], x1 = acc[iu][ju][1], x2 = acc[iu][ju][2], x3 = acc[iu][ju][3];
            fmac_asm(x0, p[0], sc[iu][0]);
            fmac_asm(x1, p[1], sc[iu][TR ? 0 : 1]);
            fmac_asm(x2, p[2], sc[iu][TR ? 0 : 2]);
            fmac_asm(x3, p[3], sc[iu][TR ? 0 : 3]);
            acc[iu][ju] = v4f{x0, x1, x2, x3};
        }
    }
#pragma unroll
    for (int q = 0; q < 3; q++)
#pragma unroll
        for (int r = 0; r < (TR ? 1 : 4); r++) scp[q][r] = sc[1 + q][r];  // the last three MFMAs: row tiles 1-3
}

// The K step of a wave of a partial last row tile whose rows below M fill only its first TMV < 4 row tiles of 16:
// those row tiles' MFMAs and promotions, with the operands, order of promotion and instructions bs_step_fixed uses
// for them (so their accumulators are bit-identical), the others left at zero as the zero rows past M would leave
// them. The stage's loads go out first, all at once.
template <class C, int TMV, bool TR = false>
__device__ __forceinline__ void bs_step_rows(const uint8_t *st, int wm0, int wn0, v4f (&acc)[C::TM][C::TN],
                                             const BsOperands<C> &op, uint32_t dstage, int dkb)
{
    static_assert(C::TM == 4 && (C::TN == 8 || C::TN == 4) && TMV >= 1 && TMV < 4,
                  "partial row tiles of 64 x 128 and 64 x 64 wave tiles");
    constexpr int LAG = 3, NM = C::TN * TMV;
    if (dkb >= 0) op.issue(dstage, dkb);
    const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
    const uint8_t *ta = st, *tb = st + C::A_BYTES;
    const float *ts = (const float *)(st + C::A_BYTES + C::B_BYTES);
    v8i a[TMV], b[3];
    b[0] = ld_frag(tb, wn0);
    b[1] = ld_frag(tb, wn0 + 16);
#pragma unroll
    for (int i = 0; i < TMV; i++) a[i] = ld_frag(ta, wm0 + 16 * i);
    const float swv = *(const float *)(st + C::A_BYTES + C::B_BYTES + C::S_BYTES + 4 * (wn0 >> 7));
    float sc[TMV][4];
#pragma unroll
    for (int i = 0; i < TMV; i++) {
        if constexpr (TR) {
            sc[i][0] = ts[wm0 + 16 * i + c16] * swv;
        } else {
            const float4 s4 = *(const float4 *)(ts + wm0 + 16 * i + 4 * g);
            sc[i][0] = s4.x * swv; sc[i][1] = s4.y * swv; sc[i][2] = s4.z * swv; sc[i][3] = s4.w * swv;
        }
    }
    v4f pr[LAG + 1];
#pragma unroll
    for (int t = 0; t < NM + LAG; t++) {
        if (t < NM) {
            const int j = t / TMV, i = t % TMV;
            if constexpr (TR) mfma_asm(pr[t % (LAG + 1)], b[j % 3], a[i]);
            else mfma_asm(pr[t % (LAG + 1)], a[i], b[j % 3]);
            if (i == 0 && j + 2 < C::TN) b[(j + 2) % 3] = ld_frag(tb, wn0 + 16 * (j + 2));
        }
        if (t == LAG) asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");  // an XDL result is read 11+ slots later
        if (t >= LAG) {
            const int u = t - LAG, j = u / TMV, i = u % TMV;
            const v4f p = pr[u % (LAG + 1)];
            float x0 = acc[i][j][0], x1 = acc[i][j][1], x2 = acc[i][j][2], x3 = acc[i][j][3];
            fmac_asm(x0, p[0], sc[i][0]);
            fmac_asm(x1, p[1], sc[i][TR ? 0 : 1]);
            fmac_asm(x2, p[2], sc[i][TR ? 0 : 2]);
            fmac_asm(x3, p[3], sc[i][TR ? 0 : 3]);
            acc[i][j] = v4f{x0, x1, x2, x3};
        }
    }
}

// Kernel arguments first used after the main loop (epilogue outputs) are read by scalar loads the compiler may leave in
// flight up to the loop. Scalar loads complete out of order, so with one pending at the loop header the compiler can
// no longer count LDS reads exactly and waits for every fragment read of a step (lgkmcnt(0)) before its first MFMA.
// Naming the arguments here, before the loop, makes the compiler load them and wait for the loads first.
template <class T>
__device__ __forceinline__ void arg_resident(T a)
{
    asm volatile("" ::"s"(a));
}
template <class... T>
__device__ __forceinline__ void args_resident(T... a)
{
    (arg_resident(a), ...);
}

struct BsNoPre {
    __device__ __forceinline__ void operator()() const {}
};

// Main loop (SKIP: waves whose rows are all past M skip their matrix work). On return acc[i][j][r] holds output row m0 + wm0 + 16 i + 4 (lane >> 4) + r, column
// n0 + wn0 + 16 j + (lane & 15), where (wm0, wn0) = bs_wave_origin(); with TR the tile transposed (the MFMAs take
// the weights as A): row m0 + wm0 + 16 i + (lane & 15), column n0 + wn0 + 16 j + 4 (lane >> 4) + r, one row scale
// per lane and row tile. The block is synchronised, no load is in
// flight and the whole shared memory is free for the epilogue. pre() runs once the first stages' loads are issued
// (epilogue inputs can be fetched there, under the prologue's memory latency); it may write shared memory only past
// C::LDS.
template <class C, class Pre = BsNoPre, bool SKIP = true, bool TR = false>
__device__ __forceinline__ void bs_mainloop(const uint8_t *__restrict__ A, int lda, const float *__restrict__ sa,
                                            int lds, const uint8_t *__restrict__ W, const float *__restrict__ sw,
                                            int M, int Npad, int K, int m0, int n0, uint8_t *smem,
                                            v4f (&acc)[C::TM][C::TN], Pre pre = Pre(), int Nlive = -1)
{
    BsOperands<C> op;
    const int KB = K >> 7;
    int wm0, wn0;
    bs_wave_origin<C>(wm0, wn0);
    op.init(A, lda, sa, lds, W, sw, K, M, Npad, m0, n0);
    const uint32_t base = lds_addr(smem);

#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int j = 0; j < C::TN; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int s = 0; s < C::NS - 1; s++)
        if (s < KB) op.issue(base + s * C::STAGE, s);
    pre();
    // rows of this wave below M (wave-uniform): in a partial last row tile a wave runs only the row tiles of 16 that
    // hold such rows (a wave with none only issues its share of the loads); accumulators it skips stay zero, as the
    // zero rows past M would leave them
    // (a wave whose columns all lie at or past Nlive, the first column that is zero padding throughout, is dead too)
    const int live = !SKIP ? C::WM
                     : __builtin_amdgcn_readfirstlane(n0 + wn0) >= (Nlive < 0 ? Npad : Nlive) ? 0
                                                                                               : M - __builtin_amdgcn_readfirstlane(m0 + wm0);
    // the K loop around one kind of step (each kind runs its own copy of the loop, so their registers never meet)
    auto kloop = [&](auto step) {
        int cs = 0, is = C::NS - 1;  // stage computed now, stage issued now
        for (int kb = 0; kb < KB; kb++) {
            // stage kb must be resident; the min(NS - 2, KB - 1 - kb) stages issued after it may stay in flight
            if (kb + C::NS - 2 < KB) wait_vmem_n<(C::NS - 2) * C::LPS>();
            else wait_vmem();
            lds_barrier();  // every wave's part of stage kb landed; every wave finished reading stage kb - 1
            step(smem + cs * C::STAGE, base + is * C::STAGE, kb + C::NS - 1 < KB ? kb + C::NS - 1 : -1);
            cs = cs == C::NS - 1 ? 0 : cs + 1;
            is = is == C::NS - 1 ? 0 : is + 1;
        }
    };
    if constexpr (C::TM == 4 && (C::TN == 8 || C::TN == 4)) {
        if (live > 32) {
            v4f pr[4];          // the MFMA result ring, and the scales of the last step's MFMAs 29-31 (their
            float scp[3][4];    // promotions run at the start of the next step)
            int kbi = 0;
            kloop([&](const uint8_t *st, uint32_t dst, int dkb) {
                bs_step_fixed<C, TR>(st, wm0, wn0, acc, op, dst, dkb, pr, scp, kbi > 0);
                kbi++;
            });
            asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");  // 12+ wait states after the last MFMA
            bs_step_fixed_flush<C, TR>(acc, pr, scp);
        } else if (live > 16)
            kloop([&](const uint8_t *st, uint32_t dst, int dkb) {
                bs_step_rows<C, 2, TR>(st, wm0, wn0, acc, op, dst, dkb);
            });
        else if (live > 0)
            kloop([&](const uint8_t *st, uint32_t dst, int dkb) {
                bs_step_rows<C, 1, TR>(st, wm0, wn0, acc, op, dst, dkb);
            });
        else
            kloop([&](const uint8_t *, uint32_t dst, int dkb) {
                if (dkb >= 0) op.issue(dst, dkb);
            });
    } else {
        static_assert(!TR, "the transposed tile needs the fixed-order steps");
        kloop([&](const uint8_t *st, uint32_t dst, int dkb) {
            if (dkb >= 0) op.issue(dst, dkb);
            bs_step<C>(st, wm0, wn0, acc);
        });
    }
    lds_barrier();
}

// ---- 2:4-sparse weights ----------------------------------------------------------------------------------------
// W is stored compressed (xtagger_amd pack24 layout): for 16-row tile t and K block kb, 64 lanes l = 16 g + r hold
// row 16 t + r, dense k in [128 kb + 32 g, +32) as 16 value bytes (2 of every 4) in vals [N/16][K/128][64][16] and one
// index word (nibble j = p0 | p1 << 2 for group j) in idx [N/16][K/128][64]. v_smfmac_f32_16x16x128_fp8_fp8 takes the
// sparse operand as A with exactly that lane layout, and the dense operand (the activations) as B in the layout
// ld_frag reads: lane group g of B holds chunks g and g + 4 of its row, which makes sparse lane group g cover dense k
// [32 g, 32 g + 32) of the same 128-wide block (measured on gfx950 for every group and index pattern). Each 1 KB value
// block and 256-byte index block is contiguous in memory and in LDS, read lane-linear.
// A wave computes the transposed tile D'[n][m] (weight rows as MFMA rows), promoted per K block with the activation
// scale of its column m and the weight-block scale; bs_sp_to_dense then moves it into the dense accumulator layout.

template <class C>
struct BsSpOperands {
    v4i ra, rv, rx, rs;
    uint32_t a_off[C::LA], v_off[C::LV], x_off[C::LV], s_off;
    uint32_t s_step;
    uint32_t m0_a, m0_v, m0_x, m0_s;

    __device__ __forceinline__ void init(const uint8_t *A, int lda, const float *sa, int lds, const uint8_t *V,
                                         const uint32_t *X, const float *sw, int K, int M, int Npad, int m0, int n0)
    {
        const int KB = K >> 7, NT16 = Npad >> 4;
        ra = buf_desc(A, (uint32_t)M * (uint32_t)lda);
        rv = buf_desc(V, (uint32_t)NT16 * (uint32_t)KB * 1024u);
        rx = buf_desc(X, (uint32_t)NT16 * (uint32_t)KB * 256u);
        const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
        const int r8 = lane >> 3, p = lane & 7;
#pragma unroll
        for (int i = 0; i < C::LA; i++) {
            const int rl = 8 * (w * C::LA + i) + r8, m = m0 + rl;
            a_off[i] = m < M ? (uint32_t)m * (uint32_t)lda + (uint32_t)(((p - rl) & 7) << 4) : XT_OOR;
        }
#pragma unroll
        for (int i = 0; i < C::LV; i++) {
            const int t = (n0 >> 4) + w * C::LV + i;
            v_off[i] = t < NT16 ? (uint32_t)t * (uint32_t)KB * 1024u + 16u * lane : XT_OOR;
            x_off[i] = t < NT16 ? (uint32_t)t * (uint32_t)KB * 256u + 4u * lane : XT_OOR;
        }
        m0_a = (uint32_t)(1024 * w * C::LA);
        m0_v = (uint32_t)(C::A_BYTES + 1024 * w * C::LV);
        m0_x = (uint32_t)(C::A_BYTES + C::V_BYTES + 256 * w * C::LV);
        if (w < C::SL) {
            rs = buf_desc(sa, (uint32_t)KB * (uint32_t)lds * 4u);
            const int m = m0 + 64 * w + lane;
            s_off = m < lds ? (uint32_t)m * 4u : XT_OOR;
            s_step = (uint32_t)lds * 4u;
            m0_s = (uint32_t)(C::A_BYTES + C::V_BYTES + C::X_BYTES + 256 * w);
        } else {
            const int nbt = Npad >> 7, nb = (n0 >> 7) + lane;
            rs = buf_desc(sw, (uint32_t)nbt * (uint32_t)KB * 4u);
            s_off = (lane < C::BN / 128 && nb < nbt) ? (uint32_t)(nb * KB) * 4u : XT_OOR;
            s_step = 4u;
            m0_s = (uint32_t)(C::A_BYTES + C::V_BYTES + C::X_BYTES + C::S_BYTES);
        }
    }

    __device__ __forceinline__ void issue(uint32_t stage, int kb) const
    {
#pragma unroll
        for (int i = 0; i < C::LA; i++) dma16(ra, stage + m0_a + 1024u * i, a_off[i], (uint32_t)kb * 128u);
#pragma unroll
        for (int i = 0; i < C::LV; i++) dma16(rv, stage + m0_v + 1024u * i, v_off[i], (uint32_t)kb * 1024u);
#pragma unroll
        for (int i = 0; i < C::LV; i++) dma4(rx, stage + m0_x + 256u * i, x_off[i], (uint32_t)kb * 256u);
        dma4(rs, stage + m0_s, s_off, (uint32_t)kb * s_step);
    }
    // load q (0 .. LPS_SP - 1) of K step kb: the same loads as issue(), one at a time
    __device__ __forceinline__ void issue_one(int q, uint32_t stage, int kb) const
    {
        if (q < C::LA) dma16(ra, stage + m0_a + 1024u * q, a_off[q], (uint32_t)kb * 128u);
        else if (q < C::LA + C::LV) dma16(rv, stage + m0_v + 1024u * (q - C::LA), v_off[q - C::LA], (uint32_t)kb * 1024u);
        else if (q < C::LA + 2 * C::LV)
            dma4(rx, stage + m0_x + 256u * (q - C::LA - C::LV), x_off[q - C::LA - C::LV], (uint32_t)kb * 256u);
        else dma4(rs, stage + m0_s, s_off, (uint32_t)kb * s_step);
    }
};

// One K step: TN x TM sparse MFMAs into the transposed accumulators accT[n tile][m tile], in a fixed issue order (the
// dense step's: single-instruction asm for the matrix instructions and the promotion fmas, every LDS read between
// them). MFMA t = 4 j + i takes weight tile j (values and indices, a 3-slot ring: tile j + 2 is read after MFMA
// (j, 0)) and activation tile i; its partial is promoted after MFMA t + 3, from a ring of 6. v_smfmac's accumulator
// is tied to its destination, so every partial must start from zeros: the slot a promotion frees is refilled for
// MFMA t + 6 by a broadcast read of 16 zero bytes of shared memory (zl), two MFMAs ahead of its use, which takes
// two VALU moves per MFMA off the step (VALU bound here: the sparse MFMA runs in half the dense one's cycles while
// the promotion keeps its four fmas). 2.4% off the sparse layer step at M=8200 against the compiler's order with
// moves; the ring of 5 (the read one MFMA ahead) gained 1.7-2.0%, 7 gained 2.0%, and 8 leaves no registers to spare.
// The LPS_SP loads of K step dkb (dkb < 0: none) go out one per MFMA from MFMA 1 on.
__device__ __forceinline__ void smfmac_asm(v4f &p, const v4i &w, const v8i &x, int idx)
{
    asm volatile("v_smfmac_f32_16x16x128_fp8_fp8 %0, %1, %2, %3" : "+v"(p) : "v"(w), "v"(x), "v"(idx) : "memory");
}
// p = 0 here, loaded from 16 zero bytes of shared memory (zl: byte offset): a broadcast LDS read in place of two
// VALU moves. The load is volatile, so each partial gets its own and keeps its registers until its MFMA.
typedef __attribute__((address_space(3))) const v4f lds_v4f;
__device__ __forceinline__ void lds_zero(v4f &p, uint32_t zl)
{
    p = *(volatile lds_v4f *)(uintptr_t)zl;
}

template <class C>
__device__ __forceinline__ void bs_step_sp(const uint8_t *st, int wm0, int wn0, v4f (&accT)[C::TN][C::TM],
                                           const BsSpOperands<C> &op, uint32_t dstage, int dkb, uint32_t zl)
{
    static_assert(C::TM == 4 && C::TN >= 2 && C::LPS_SP < C::TN * C::TM, "schedule written for 64-row wave tiles");
    const int lane = threadIdx.x & 63, c16 = lane & 15;
    const uint8_t *ta = st, *tv = st + C::A_BYTES, *tx = st + C::A_BYTES + C::V_BYTES;
    const float *ts = (const float *)(st + C::A_BYTES + C::V_BYTES + C::X_BYTES);
    // the wave's weight tiles j = 0 .. TN - 1 at tvl + 1024 j and txl + 256 j (constant offsets of one base each)
    const uint8_t *tvl = tv + (wn0 >> 4) * 1024 + 16 * lane, *txl = tx + (wn0 >> 4) * 256 + 4 * lane;
    constexpr int NS = C::TN * C::TM, LAG = 3, R = 6;
    v4i v[3];
    int x[3];
    v8i xa[4];
    v[0] = *(const v4i *)tvl;
    x[0] = *(const int *)txl;
    xa[0] = ld_frag(ta, wm0);
    asm volatile("" ::: "memory");  // the first MFMA waits for these reads only
    const float swv = *(const float *)(st + C::A_BYTES + C::V_BYTES + C::X_BYTES + C::S_BYTES + 4 * (wn0 >> 7));
    float sr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) sr[i] = ts[wm0 + 16 * i + c16];
    asm volatile("" ::: "memory");
    xa[1] = ld_frag(ta, wm0 + 16);
    xa[2] = ld_frag(ta, wm0 + 32);
    xa[3] = ld_frag(ta, wm0 + 48);
    v[1] = *(const v4i *)(tvl + 1024);
    x[1] = *(const int *)(txl + 256);
    asm volatile("" ::: "memory");
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) sc[i] = sr[i] * swv;
    v4f pr[R];
#pragma unroll
    for (int r = 0; r < R; r++) lds_zero(pr[r], zl);
#pragma unroll
    for (int t = 0; t < NS + LAG; t++) {
        if (t < NS) {
            const int j = t >> 2, i = t & 3;
            smfmac_asm(pr[t % R], v[j % 3], xa[i], x[j % 3]);
            if (i == 0 && j + 2 < C::TN) {
                v[(j + 2) % 3] = *(const v4i *)(tvl + 1024 * (j + 2));
                x[(j + 2) % 3] = *(const int *)(txl + 256 * (j + 2));
            }
            if (t >= 1 && t <= C::LPS_SP && dkb >= 0) op.issue_one(t - 1, dstage, dkb);
        }
        if (t == LAG) asm volatile("s_nop 7" ::: "memory");
        if (t >= LAG) {
            const int u = t - LAG, ju = u >> 2, iu = u & 3;
            const v4f p = pr[u % R];
            float x0 = accT[ju][iu][0], x1 = accT[ju][iu][1], x2 = accT[ju][iu][2], x3 = accT[ju][iu][3];
            fmac_asm(x0, p[0], sc[iu]);
            fmac_asm(x1, p[1], sc[iu]);
            fmac_asm(x2, p[2], sc[iu]);
            fmac_asm(x3, p[3], sc[iu]);
            accT[ju][iu] = v4f{x0, x1, x2, x3};
            if (u + R < NS) lds_zero(pr[u % R], zl);  // for MFMA u + 6
        }
    }
}

// The transposed wave tile (accT[n tile][m tile][r]: n = wn0 + 16 i + 4 (lane >> 4) + r, m = wm0 + 16 j + (lane & 15))
// to the dense accumulator layout of bs_mainloop, through the wave's own 64 x 68 fp32 slice of shared memory
// (slices at `slices` + wave * 17408 bytes), 64 columns per pass.
template <class C>
__device__ __forceinline__ void bs_sp_to_dense(uint8_t *slices, v4f (&accT)[C::TN][C::TM], v4f (&acc)[C::TM][C::TN])
{
    static_assert(C::TM == 4 && C::TN % 4 == 0, "64-row wave tiles, whole 64-column passes");
    float *tr = (float *)(slices + (threadIdx.x >> 6) * (64 * 68 * 4));
    const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15;
#pragma unroll
    for (int pass = 0; pass < C::TN / 4; pass++) {
        if (pass) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                *(float4 *)(tr + (16 * j + c16) * 68 + 16 * i + 4 * g) =
                    make_float4(accT[4 * pass + i][j][0], accT[4 * pass + i][j][1], accT[4 * pass + i][j][2],
                                accT[4 * pass + i][j][3]);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slice is the wave's own: no block barrier needed
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[i][4 * pass + j][r] = tr[(16 * i + 4 * g + r) * 68 + 16 * j + c16];
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// Sparse main loop: the same contract as bs_mainloop (dense accumulator layout on return, block synchronised, no load
// in flight, shared memory free), with the weights given as pack24 values V and indices X plus the dense 128 x 128
// block scales sw. Uses LDS_SP bytes of shared memory during the K loop and NW * 17408 bytes at the end for the
// transposition. SPREAD: the next stage's loads go out one per MFMA (bs_step_sp); otherwise in a burst after the
// barrier. Spreading them needs K known at compile time: with K a kernel argument the per-load branches of the last
// step cost the 256 x 256 tile ~40 VGPRs of spills.
// bs_mainloop_sp_t stops before the transposition: it leaves the wave's tile in accT (accT[n tile][m tile][r]:
// n = wn0 + 16 i + 4 (lane >> 4) + r, m = wm0 + 16 j + (lane & 15)), block synchronised, no load in flight, shared
// memory free, for an epilogue that reads that layout instead of paying bs_sp_to_dense's pass through shared memory.
template <class C, class Pre = BsNoPre, bool SPREAD = true>
__device__ __forceinline__ void bs_mainloop_sp_t(const uint8_t *__restrict__ A, int lda, const float *__restrict__ sa,
                                                 int lds, const uint8_t *__restrict__ V, const uint32_t *__restrict__ X,
                                                 const float *__restrict__ sw, int M, int Npad, int K, int m0, int n0,
                                                 uint8_t *smem, v4f (&accT)[C::TN][C::TM], Pre pre = Pre(),
                                                 int Nlive = -1)
{
    BsSpOperands<C> op;
    const int KB = K >> 7;
    int wm0, wn0;
    bs_wave_origin<C>(wm0, wn0);
    op.init(A, lda, sa, lds, V, X, sw, K, M, Npad, m0, n0);
    const uint32_t base = lds_addr(smem);
#pragma unroll
    for (int i = 0; i < C::TN; i++)
#pragma unroll
        for (int j = 0; j < C::TM; j++) accT[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < C::NS - 1; s++)
        if (s < KB) op.issue(base + s * C::STAGE_SP, s);
    // 16 zero bytes past the stages, published by the K loop's first barrier: every partial starts from them
    const uint32_t zl = base + C::NS * C::STAGE_SP;
    if (threadIdx.x < 4) ((float *)(smem + C::NS * C::STAGE_SP))[threadIdx.x] = 0.f;
    pre();
    // a wave whose rows are all past M skips its matrix work (accumulators stay zero)
    const bool live = __builtin_amdgcn_readfirstlane(m0 + wm0) < M &&
                      __builtin_amdgcn_readfirstlane(n0 + wn0) < (Nlive < 0 ? Npad : Nlive);
    int cs = 0, is = C::NS - 1;
    for (int kb = 0; kb < KB; kb++) {
        if (kb + C::NS - 2 < KB) wait_vmem_n<(C::NS - 2) * C::LPS_SP>();
        else wait_vmem();
        lds_barrier();
        const int dkb = kb + C::NS - 1 < KB ? kb + C::NS - 1 : -1;
        if constexpr (SPREAD) {
            if (live) bs_step_sp<C>(smem + cs * C::STAGE_SP, wm0, wn0, accT, op, base + is * C::STAGE_SP, dkb, zl);
            else if (dkb >= 0) op.issue(base + is * C::STAGE_SP, dkb);
        } else {
            if (dkb >= 0) op.issue(base + is * C::STAGE_SP, dkb);
            if (live) bs_step_sp<C>(smem + cs * C::STAGE_SP, wm0, wn0, accT, op, 0u, -1, zl);
        }
        cs = cs == C::NS - 1 ? 0 : cs + 1;
        is = is == C::NS - 1 ? 0 : is + 1;
    }
    lds_barrier();
}

template <class C, class Pre = BsNoPre, bool SPREAD = true>
__device__ __forceinline__ void bs_mainloop_sp(const uint8_t *__restrict__ A, int lda, const float *__restrict__ sa,
                                               int lds, const uint8_t *__restrict__ V, const uint32_t *__restrict__ X,
                                               const float *__restrict__ sw, int M, int Npad, int K, int m0, int n0,
                                               uint8_t *smem, v4f (&acc)[C::TM][C::TN], Pre pre = Pre(),
                                               int Nlive = -1)
{
    v4f accT[C::TN][C::TM];
    bs_mainloop_sp_t<C, Pre, SPREAD>(A, lda, sa, lds, V, X, sw, M, Npad, K, m0, n0, smem, accT, pre, Nlive);
    bs_sp_to_dense<C>(smem, accT, acc);
    lds_barrier();
}

// XCD-aware tile order for a 1-D grid of T = tiles_m * tiles_n blocks. Blocks are dispatched to the 8 XCDs round
// robin (block b -> XCD x = b % 8), so XCD x runs c_x = T / 8 + (x < T % 8) blocks. When the last row tile is partial
// (rows past M), its tiles_n tiles cost far less than a full tile (the waves past M skip their matrix work), so the
// Tf = T - tiles_n full tiles are dealt out evenly first, f_x = Tf / 8 + (x < Tf % 8) to XCD x, and the partial tiles
// take the c_x - f_x >= 0 remaining slots, at the start of each XCD's sequence: a whole extra full tile never lands on
// an XCD whose CUs already run as many as the others. Each XCD's full tiles are a contiguous run of a grouped raster
// (XT_GM row tiles walked together across all column tiles): the blocks an XCD runs at once share a few A row tiles
// and W column tiles in that XCD's L2.
__device__ __forceinline__ void tile_of_block(int tiles_m, int tiles_n, bool partial, int &tm, int &tn)
{
    const int T = tiles_m * tiles_n, Tf = partial ? T - tiles_n : T, b = blockIdx.x, x = b & 7, k = b >> 3;
    const int q = T >> 3, r = T & 7, qf = Tf >> 3, rf = Tf & 7;
    const int npx = (q + (x < r)) - (qf + (x < rf));
    if (k < npx) {
        tm = tiles_m - 1;
        tn = x * (q - qf) + (x < r ? x : r) - (x < rf ? x : rf) + k;
        return;
    }
    const int pos = x * qf + (x < rf ? x : rf) + (k - npx), tmf = partial ? tiles_m - 1 : tiles_m;
    const int per_group = XT_GM * tiles_n, grp = pos / per_group, rem = pos - grp * per_group;
    const int gm = tmf - grp * XT_GM < XT_GM ? tmf - grp * XT_GM : XT_GM;
    tm = grp * XT_GM + rem % gm;
    tn = rem / gm;
}
