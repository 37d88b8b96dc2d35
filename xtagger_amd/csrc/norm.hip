// norm.hip - bandwidth-bound kernels around the block GEMMs: LayerNorm -> E4M3 with 1x128 scales (k_ln,
// src/engine/kern_common.cuh:147-186), the mean-pool over patch tokens (k_pool, src/engine/eva_kernels.cu:402-431)
// and the final LayerNorm -> fp16 head input -> E4M3 (k_lnh, kern_common.cuh:188-192).
//
// One wave64 per 1024-wide row: lane l owns elements [8l, 8l+8) and [512+8l, 512+8l+8), so every load is a
// 16-byte coalesced access and each 128-element scale block is 16 aligned lanes. Sums run per lane in element
// order, then through an xor butterfly (32, 16, ..., 1), a fixed order the host restatement follows exactly.
#include "xt_abi.h"
#include "xt_common.h"

// LayerNorm of one row held as v[16] (lane layout above), eps 1e-6 (the blocks; 1e-5 for the PixAI head), two-pass:
// y = fma((x - mean) * rstd, gamma, beta), rstd = 1 / sqrt(var + eps) with IEEE sqrt and division. gg / bb hold the
// lane's 16 gamma / beta values in the same layout.
__device__ __forceinline__ void ln16_gb(float *v, const float *gg, const float *bb, float eps = XT_EPS)
{
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 16; j++) s += v[j];
    const float mean = wave_sum(s) * (1.0f / 1024.0f);
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const float d = v[j] - mean;
        q = __builtin_fmaf(d, d, q);
    }
    const float var = wave_sum(q) * (1.0f / 1024.0f);
    const float rstd = 1.0f / __builtin_sqrtf(var + eps);
#pragma unroll
    for (int j = 0; j < 16; j++) v[j] = __builtin_fmaf((v[j] - mean) * rstd, gg[j], bb[j]);
}

// the lane's 16 values of a 1024-float vector (gamma or beta) in the row layout
__device__ __forceinline__ void load_vec16(const float *__restrict__ g, int lane, float *gg)
{
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const float4 g0 = *(const float4 *)(g + 512 * h + 8 * lane), g1 = *(const float4 *)(g + 512 * h + 8 * lane + 4);
        gg[8 * h + 0] = g0.x; gg[8 * h + 1] = g0.y; gg[8 * h + 2] = g0.z; gg[8 * h + 3] = g0.w;
        gg[8 * h + 4] = g1.x; gg[8 * h + 5] = g1.y; gg[8 * h + 6] = g1.z; gg[8 * h + 7] = g1.w;
    }
}

__device__ __forceinline__ void ln16(float *v, const float *__restrict__ g, const float *__restrict__ b, int lane,
                                     float eps = XT_EPS)
{
    float gg[16], bb[16];
    load_vec16(g, lane, gg);
    load_vec16(b, lane, bb);
    ln16_gb(v, gg, bb, eps);
}

// v[16] -> E4M3 bytes of the row at q (row-major, 1024 bytes) and its 8 scales at s[kb * lds + row]
__device__ __forceinline__ void quant_row16(const float *v, uint8_t *__restrict__ q, float *__restrict__ s, int lds,
                                            int row, int lane)
{
#pragma unroll
    for (int h = 0; h < 2; h++) {
        float amax = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[8 * h + j]));
        amax = row16_absmax(amax);  // the 16 lanes of the block: one DPP row
        const float sc = block_scale(amax), inv = block_scale_inv(sc);
        const float *w = v + 8 * h;
        uint2 o;
        o.x = e4_pack4_scaled(w[0] * inv, w[1] * inv, w[2] * inv, w[3] * inv);
        o.y = e4_pack4_scaled(w[4] * inv, w[5] * inv, w[6] * inv, w[7] * inv);
        *(uint2 *)(q + 512 * h + 8 * lane) = o;
        if ((lane & 15) == 0) s[(size_t)(4 * h + (lane >> 4)) * lds + row] = sc;
    }
}

// the lane's 2 x 16 bytes of a 1024-half row, and their conversion to v[16]
__device__ __forceinline__ void load_raw16(const uint16_t *__restrict__ x, int lane, uint4 (&u)[2])
{
    u[0] = *(const uint4 *)(x + 8 * lane);
    u[1] = *(const uint4 *)(x + 512 + 8 * lane);
}
__device__ __forceinline__ void unpack16_f16(const uint4 (&u)[2], float *v)
{
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t w[4] = {u[h].x, u[h].y, u[h].z, u[h].w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[8 * h + 2 * i] = h2f((uint16_t)(w[i] & 0xffffu));
            v[8 * h + 2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
        }
    }
}
__device__ __forceinline__ void load_row16_f16(const uint16_t *__restrict__ x, int lane, float *v)
{
    uint4 u[2];
    load_raw16(x, lane, u);
    unpack16_f16(u, v);
}

// k_ln: x fp16 [rows][1024] -> q E4M3 [rows][1024] + s [8][lds]. The grid is as many 256-thread blocks as stay
// resident at once (LN_WAVES_PER_SIMD waves per SIMD on every CU, or fewer blocks for short inputs); wave w of its W
// waves takes rows w, w + W, w + 2W, ..., so the waves in flight work on W consecutive rows at a time. A wave loads
// gamma and beta once and holds them in registers (8 KB of reads per row otherwise; 3% of the kernel's time), and
// issues the next row's 2 KB load before it normalises the current row.
#define LN_WAVES_PER_SIMD 6
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(LN_WAVES_PER_SIMD, 8)))
k_ln(const uint16_t *__restrict__ x, const float *__restrict__ g, const float *__restrict__ b, uint8_t *__restrict__ q,
     float *__restrict__ s, int rows, int lds)
{
    const int lane = threadIdx.x & 63, W = (int)gridDim.x * 4;
    int row = (int)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    // rows are read through a descriptor that ends at row `rows`: the prefetch past the last row loads zeros and
    // touches no memory, so it needs no branch (rows <= 2^19: every offset fits 32 bits)
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, (uint32_t)rows * (XT_D * 2u));
    auto load = [&](int r, uint4 (&u)[2]) {
        const uint32_t o = (uint32_t)r * (XT_D * 2u) + 16u * (uint32_t)lane;
        u[0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)o, 0, 0));
        u[1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(o + 1024u), 0, 0));
    };
    uint4 cur[2];
    load(row, cur);
    float gg[16], bb[16];
    load_vec16(g, lane, gg);
    load_vec16(b, lane, bb);
    // wait for gamma and beta here, once: left to the loop, the waits for them (taken as counts of the memory
    // operations issued since) would stall every row on the next row's prefetch and this row's stores
#pragma unroll
    for (int j = 0; j < 16; j++) asm volatile("" : "+v"(gg[j]), "+v"(bb[j]));
    for (;;) {
        const int nrow = row + W;  // rows < 2^19 and W < 2^20: no overflow
        uint4 nxt[2];
        load(nrow < rows ? nrow : rows, nxt);
        __builtin_amdgcn_sched_barrier(0);  // the prefetch goes out before this row's work, not sunk into it
        float v[16];
        unpack16_f16(cur, v);
        ln16_gb(v, gg, bb);
        quant_row16(v, q + (size_t)row * XT_D, s, lds, row, lane);
        if (nrow >= rows) break;
        row = nrow;
        cur[0] = nxt[0];
        cur[1] = nxt[1];
    }
}

// k_pool: mean over tokens 1..1024 of each image: x fp16 [nb * 1025][1024] -> p fp32 [nb][1024]. Grid (nb, 8) of
// 512 threads, 128 columns per block: thread (g, c) = (t >> 4, t & 15) sums tokens 1 + 32 g .. 32 g + 32 of columns
// 8 c .. 8 c + 7 in token order, one 16-byte load per token; a column's 32 group sums then meet in group order
// through shared memory, and the total is scaled by 1/1024.
__global__ void __launch_bounds__(512) k_pool(const uint16_t *__restrict__ x, float *__restrict__ p)
{
    __shared__ __attribute__((aligned(16))) float red[32][128 + 4];
    const int c = threadIdx.x & 15, g = threadIdx.x >> 4, col0 = blockIdx.y * 128;
    const uint16_t *xr = x + ((size_t)blockIdx.x * XT_T + 1 + 32 * g) * XT_D + col0 + 8 * c;
    float s[8];
#pragma unroll
    for (int k = 0; k < 8; k++) s[k] = 0.f;
#pragma unroll 8
    for (int t = 0; t < 32; t++) {
        const uint4 u = *(const uint4 *)(xr + (size_t)t * XT_D);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            s[2 * k] += h2f((uint16_t)(w[k] & 0xffffu));
            s[2 * k + 1] += h2f((uint16_t)(w[k] >> 16));
        }
    }
    *(float4 *)&red[g][8 * c] = make_float4(s[0], s[1], s[2], s[3]);
    *(float4 *)&red[g][8 * c + 4] = make_float4(s[4], s[5], s[6], s[7]);
    __syncthreads();
    if (threadIdx.x < 128) {
        float a = red[0][threadIdx.x];
#pragma unroll 8
        for (int i = 1; i < 32; i++) a += red[i][threadIdx.x];
        p[(size_t)blockIdx.x * XT_D + col0 + threadIdx.x] = a * (1.0f / XT_NP);
    }
}

// k_lnh: final LayerNorm of the pooled rows (fc_norm) -> fp16 head input pn [nb][1024] (the reference's head
// operand, also read back as hpn), then E4M3 of those fp16 values with 1x128 scales for the FP8 head.
__global__ void __launch_bounds__(256) k_lnh(const float *__restrict__ p, const float *__restrict__ g,
                                             const float *__restrict__ b, uint16_t *__restrict__ pn,
                                             uint8_t *__restrict__ q, float *__restrict__ s, int rows, int lds)
{
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    float v[16];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const float4 a = *(const float4 *)(p + (size_t)row * XT_D + 512 * h + 8 * lane);
        const float4 c = *(const float4 *)(p + (size_t)row * XT_D + 512 * h + 8 * lane + 4);
        v[8 * h + 0] = a.x; v[8 * h + 1] = a.y; v[8 * h + 2] = a.z; v[8 * h + 3] = a.w;
        v[8 * h + 4] = c.x; v[8 * h + 5] = c.y; v[8 * h + 6] = c.z; v[8 * h + 7] = c.w;
    }
    ln16(v, g, b, lane);
#pragma unroll
    for (int h = 0; h < 2; h++) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint16_t lo = f2h(v[8 * h + 2 * i]), hi = f2h(v[8 * h + 2 * i + 1]);
            v[8 * h + 2 * i] = h2f(lo);
            v[8 * h + 2 * i + 1] = h2f(hi);
            w[i] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        *(uint4 *)(pn + (size_t)row * XT_D + 512 * h + 8 * lane) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    quant_row16(v, q + (size_t)row * XT_D, s, lds, row, lane);
}

// k_px_pembed (px_kernels.cu:16-50 k_pembed): x = f16(LN_1e-5(x + pos[m % T]) g + b) in place, x fp16 [rows][1024]
// window-major token rows, pos fp32 [T][1024]; the position is added in fp32 to the fp16 patch embedding.
__global__ void __launch_bounds__(256) k_px_pembed(uint16_t *__restrict__ x, const float *__restrict__ pos, int T,
                                                   const float *__restrict__ g, const float *__restrict__ b, int rows)
{
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    float v[16];
    uint16_t *xr = x + (size_t)row * XT_D;
    load_row16_f16(xr, lane, v);
    const float *pr = pos + (size_t)(row % T) * XT_D;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const float4 a = *(const float4 *)(pr + 512 * h + 8 * lane), c = *(const float4 *)(pr + 512 * h + 8 * lane + 4);
        v[8 * h + 0] += a.x; v[8 * h + 1] += a.y; v[8 * h + 2] += a.z; v[8 * h + 3] += a.w;
        v[8 * h + 4] += c.x; v[8 * h + 5] += c.y; v[8 * h + 6] += c.z; v[8 * h + 7] += c.w;
    }
    ln16(v, g, b, lane, 1e-5f);
#pragma unroll
    for (int h = 0; h < 2; h++) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; i++) w[i] = (uint32_t)f2h(v[8 * h + 2 * i]) | ((uint32_t)f2h(v[8 * h + 2 * i + 1]) << 16);
        *(uint4 *)(xr + 512 * h + 8 * lane) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// k_px_hln: the PixAI attention-pool head's keys / values and scores (px_kernels.cu:344-400 k_phln + k_phscore,
// fused): y = f16(LN_1e-5(x) + hpos[m % T]) fp16 [rows][1024] and s [rows][16] = U y of the fp16 y (exp2 domain, the
// constant query folded into U). U [16][1024] fp32 sits in shared memory; each wave takes 16 rows in turn, and each
// score is the lane's 16 products in element order (an fma chain) met in the xor butterfly.
constexpr int PX_HLN_ROWS = 16;  // rows per wave
__global__ void __launch_bounds__(256) k_px_hln(const uint16_t *__restrict__ x, const float *__restrict__ g,
                                                const float *__restrict__ b, const uint16_t *__restrict__ hpos, int T,
                                                const float *__restrict__ U, uint16_t *__restrict__ y,
                                                float *__restrict__ s, int rows)
{
    __shared__ __attribute__((aligned(16))) float su[16 * XT_D];
    for (int i = threadIdx.x; i < 16 * XT_D / 4; i += 256) ((float4 *)su)[i] = ((const float4 *)U)[i];
    __syncthreads();
    const int lane = threadIdx.x & 63, r0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * PX_HLN_ROWS;
    if (r0 >= rows) return;
    // gamma and beta in registers, waited for once; each row's x and position rows are loaded while the row before
    // is worked on, through descriptors that end at row `rows` of x and row T of hpos (past them: zeros, no traffic)
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, (uint32_t)rows * (XT_D * 2u)), rh = buf_rsrc(hpos, (uint32_t)T * (XT_D * 2u));
    auto load = [&](__amdgpu_buffer_rsrc_t rsrc, int r, uint4 (&u)[2]) {
        const uint32_t o = (uint32_t)r * (XT_D * 2u) + 16u * (uint32_t)lane;
        u[0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)o, 0, 0));
        u[1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)(o + 1024u), 0, 0));
    };
    uint4 cx[2], ch[2];
    load(rx, r0, cx);
    load(rh, r0 % T, ch);
    float gg[16], bb[16];
    load_vec16(g, lane, gg);
    load_vec16(b, lane, bb);
#pragma unroll
    for (int j = 0; j < 16; j++) asm volatile("" : "+v"(gg[j]), "+v"(bb[j]));
    for (int rr = 0; rr < PX_HLN_ROWS; rr++) {
        const int row = r0 + rr;
        const bool more = rr + 1 < PX_HLN_ROWS && row + 1 < rows;
        uint4 nx[2], nh[2];
        load(rx, more ? row + 1 : rows, nx);
        load(rh, more ? (row + 1) % T : T, nh);
        __builtin_amdgcn_sched_barrier(0);  // the prefetch goes out before this row's work
        float v[16], hp[16];
        unpack16_f16(cx, v);
        unpack16_f16(ch, hp);
        ln16_gb(v, gg, bb, 1e-5f);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint16_t lo = f2h(v[8 * h + 2 * i] + hp[8 * h + 2 * i]);
                const uint16_t hi = f2h(v[8 * h + 2 * i + 1] + hp[8 * h + 2 * i + 1]);
                v[8 * h + 2 * i] = h2f(lo);
                v[8 * h + 2 * i + 1] = h2f(hi);
                w[i] = (uint32_t)lo | ((uint32_t)hi << 16);
            }
            *(uint4 *)(y + (size_t)row * XT_D + 512 * h + 8 * lane) = make_uint4(w[0], w[1], w[2], w[3]);
        }
        float mine = 0.f;
#pragma unroll
        for (int hd = 0; hd < 16; hd++) {
            float a = 0.f;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const float4 u0 = *(const float4 *)(su + hd * XT_D + 512 * h + 8 * lane);
                const float4 u1 = *(const float4 *)(su + hd * XT_D + 512 * h + 8 * lane + 4);
                const float uu[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
                for (int j = 0; j < 8; j++) a = __builtin_fmaf(uu[j], v[8 * h + j], a);
            }
            a = wave_sum(a);
            mine = lane == hd ? a : mine;
        }
        if (lane < 16) s[(size_t)row * 16 + lane] = mine;
        if (!more) break;
        cx[0] = nx[0];
        cx[1] = nx[1];
        ch[0] = nh[0];
        ch[1] = nh[1];
    }
}

int xt_cu_count()
{
    static int cu_count[64];  // per device (a benign race: every writer stores the same value)
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int cus = cu_count[dev];
    if (cus <= 0) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 0;
        cu_count[dev] = cus;
    }
    return cus;
}

// ---------------------------------------------------------------------------------------------------------------
extern "C" int eva_k_ln(const void *x, const float *g, const float *b, void *q, float *s, int rows, int lds,
                        void *stream)
{
    if (rows < 0 || lds < rows) return xt_fail("eva_k_ln", "bad shape (lds >= rows)");
    if (((uintptr_t)x | (uintptr_t)g | (uintptr_t)b | (uintptr_t)q) & 15)
        return xt_fail("eva_k_ln", "x, g, b, q must be 16-byte aligned");
    if (!rows) return 0;
    if (rows > (1 << 19)) return xt_fail("eva_k_ln", "at most 2^19 rows");
    const int cus = xt_cu_count();
    if (cus <= 0) return xt_fail("eva_k_ln", "cannot read the device's CU count");
    const int need = (rows + 3) / 4, resident = cus * LN_WAVES_PER_SIMD;  // 4 SIMDs a CU, 4 waves a block
    hipLaunchKernelGGL(k_ln, dim3(need < resident ? need : resident), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t *)x, g, b, (uint8_t *)q, s, rows, lds);
    return xt_check("eva_k_ln");
}

extern "C" int eva_k_pool(const void *x, float *p, int nb, void *stream)
{
    if (nb <= 0) return xt_fail("eva_k_pool", "nb must be positive");
    hipLaunchKernelGGL(k_pool, dim3(nb, XT_D / 128), dim3(512), 0, (hipStream_t)stream, (const uint16_t *)x, p);
    return xt_check("eva_k_pool");
}

extern "C" int eva_k_lnh(const float *p, const float *g, const float *b, void *pn, void *q, float *s, int rows,
                         int lds, void *stream)
{
    if (rows <= 0 || lds < rows) return xt_fail("eva_k_lnh", "bad shape (rows > 0, lds >= rows)");
    if (((uintptr_t)p | (uintptr_t)g | (uintptr_t)b | (uintptr_t)pn | (uintptr_t)q) & 15)
        return xt_fail("eva_k_lnh", "p, g, b, pn, q must be 16-byte aligned");
    hipLaunchKernelGGL(k_lnh, dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream, p, g, b, (uint16_t *)pn,
                       (uint8_t *)q, s, rows, lds);
    return xt_check("eva_k_lnh");
}

extern "C" int px_k_hln(const void *x, const float *g, const float *b, const void *hpos, int T, const float *U, void *y,
                        float *s, int rows, void *stream)
{
    if (rows <= 0 || T <= 0 || rows > (1 << 20) || T > (1 << 20))
        return xt_fail("px_k_hln", "bad shape (0 < rows, T <= 2^20)");
    if (((uintptr_t)x | (uintptr_t)g | (uintptr_t)b | (uintptr_t)hpos | (uintptr_t)U | (uintptr_t)y) & 15)
        return xt_fail("px_k_hln", "x, g, b, hpos, U, y must be 16-byte aligned");
    const int per = 4 * PX_HLN_ROWS;
    hipLaunchKernelGGL(k_px_hln, dim3((rows + per - 1) / per), dim3(256), 0, (hipStream_t)stream, (const uint16_t *)x,
                       g, b, (const uint16_t *)hpos, T, U, (uint16_t *)y, s, rows);
    return xt_check("px_k_hln");
}

extern "C" int px_k_pembed(void *x, const float *pos, int T, const float *g, const float *b, int rows, void *stream)
{
    if (rows <= 0 || T <= 0) return xt_fail("px_k_pembed", "bad shape (rows > 0, T > 0)");
    if (((uintptr_t)x | (uintptr_t)pos | (uintptr_t)g | (uintptr_t)b) & 15)
        return xt_fail("px_k_pembed", "x, pos, g, b must be 16-byte aligned");
    hipLaunchKernelGGL(k_px_pembed, dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream, (uint16_t *)x, pos, T, g,
                       b, rows);
    return xt_check("px_k_pembed");
}
