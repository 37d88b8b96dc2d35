// attn.hip - fused attention for EVA02-L (T = 1025 tokens, 16 heads of 64), the role of the reference's flash8
// (src/engine/kern_common.cuh:403-543) on CDNA4 bf16 matrix cores, with the output packed to E4M3 1x128 blocks
// for the out-projection.
//
// Per (image, head pair, 128-query block): 8 waves, waves 0-3 on head 2p and 4-7 on head 2p+1, 32 queries each.
// Scores are computed transposed, S^T = K Q^T (v_mfma_f32_32x32x16_bf16: A = 32 keys, B = 32 queries), so every lane
// owns one query and 16 keys of a 32-key tile. Lane group g = lane >> 5 holds accumulator rows 8j + 4g + i; the K
// fragment of lane l is read from key row pi(l & 31) with pi(8j + 4g + i) = 16(j >> 1) + 8g + 4(j & 1) + i, which
// makes accumulators 8s .. 8s+7 exactly the keys 16s + 8g .. 16s + 8g + 7: P, converted to bf16 in place, is the
// B operand of O^T += V^T P^T with V^T read as 16 contiguous bytes. No value moves between lanes.
// Softmax runs in the exp2 domain (q carries log2(e)/8 from the weights). The reference keeps a lazily refreshed
// running max so that its E4M3 weights stay below 2^8 (kern_common.cuh:480-493); bf16 weights have fp32's exponent
// range, so here each query's offset is its maximum over the first key tile and later tiles compute no maximum at all:
// the offset is raised (that tile redone from LDS) only when a weight would pass 2^64, which the tile's weight sum
// shows. l sums the bf16-rounded p that enter the PV product (the reference sums the fp32 p, kern_common.cuh:505-506):
// the output's weights then sum to one exactly, and the row sum costs one v_dot2c per pair.
// K and V^T tiles of 64 keys for both heads are double-buffered in LDS by buffer_load ... lds. The grid is 1-D and
// XCD-aware (the query blocks of one sequence and head pair run on one XCD and share its L2 copy of K and V^T), and a
// sequence of 64 n + 1 tokens takes its last key after the n tiles instead of as a tile of one key.
#include "gemm_core.h"
#include "xt_abi.h"

#define FA_QB 128                    // queries per block
#define FA_KT 64                     // keys per LDS tile
#define FA_TILE (FA_KT * 128)        // bytes of one K or V^T tile of one head
#define FA_STAGE (4 * FA_TILE)       // K head 0 | K head 1 | V^T head 0 | V^T head 1
#define FA_PLOG 64.0f                // weights stay below 2^FA_PLOG relative to the offset
#define FA_PMAX 0x1p64f

// K and V^T tiles: 128-byte rows whose 16-byte chunk c sits at c ^ ((row >> 1) & 7). A fragment read covers 16
// consecutive rows per 16 lanes (one 256-byte LDS cycle): with row bits 1-3 in the swizzle and bit 0 choosing the
// half of the 256 bytes, those rows fill all 16 slots (row & 7 alone would put rows r and r + 8 on the same banks)
__device__ __forceinline__ uint32_t swz_kv(int row, int chunk) { return (uint32_t)(row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4)); }

__device__ __forceinline__ v8bf frag_bf(const uint8_t *tile, int row, int chunk)
{
    return __builtin_bit_cast(v8bf, *(const uint4 *)(tile + swz_kv(row, chunk)));
}

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
#define kOnes2 (v2bf{(__bf16)1.0f, (__bf16)1.0f})

__device__ __forceinline__ v8bf pack_p(const v16f &s, int base)
{
    typedef float v8f __attribute__((ext_vector_type(8)));
    const v8f f = {s[base], s[base + 1], s[base + 2], s[base + 3], s[base + 4], s[base + 5], s[base + 6], s[base + 7]};
    return __builtin_convertvector(f, v8bf);
}

// One block per (query block of 128, head pair, sequence): sequences of T tokens, q / k rows and v^T columns padded to
// TP >= T rounded up to 64 (rows past T read as data must be finite; keys past T are masked). When T = 64 n + 1
// (n > 0: the wd model's 1025 tokens) the last key is not streamed as a 17th tile of one key: each lane adds it after
// the n tiles from global memory (one score, one weight, 32 products).
template <int DBG>
__global__ void __launch_bounds__(512) k_flash(const uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
                                               const uint16_t *__restrict__ vt, uint8_t *__restrict__ o8,
                                               float *__restrict__ os, int lds, float *__restrict__ o32, int T, int TP)
{
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * FA_STAGE + 8 * 32 * 4];
    float *xamax = (float *)(smem + 2 * FA_STAGE);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 5, l32 = lane & 31;
    // 1-D grid, XCD-aware: block i runs on XCD i % 8, and the query blocks of one (sequence, head pair) share its K
    // and V^T, so they all take the same i % 8 (consecutive i / 8): their K / V^T tiles are fetched into one XCD's L2
    // once instead of into every XCD's
    const int nqb = (T + FA_QB - 1) / FA_QB, bi = blockIdx.x >> 3, grp = 8 * (bi / nqb) + (blockIdx.x & 7);
    const int qb = bi - (bi / nqb) * nqb, hp = grp & (XT_NH / 2 - 1), b = grp / (XT_NH / 2);
    const int hsel = w >> 2, qt = w & 3;
    const int head = 2 * hp + hsel;
    const int q0 = qb * FA_QB + 32 * qt;
    const bool active = q0 < T;
    const bool xkey = (T & (FA_KT - 1)) == 1 && T > FA_KT;   // the last key alone, after the tiles
    const int nkt = xkey ? T / FA_KT : (T + FA_KT - 1) / FA_KT;

    // operand loads: per stage 32 x 1 KB, 4 per wave: waves 0-1 K head 2p, 2-3 K head 2p+1, 4-5 V^T head 2p, 6-7 V^T
    // head 2p+1 (K: 8 contiguous KB per head; V^T: 64 rows of 128 B, stride TP). The per-lane offsets are fixed; the
    // key tile moves only the scalar offset (8 KB of K or 128 B of V^T per tile).
    const size_t hbase0 = ((size_t)b * XT_NH + 2 * hp) * TP * XT_HD;  // elements, head 2p
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(k + hbase0, 2u * (uint32_t)TP * XT_HD * 2u);
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc(vt + hbase0, 2u * (uint32_t)TP * XT_HD * 2u);
    const int wu = __builtin_amdgcn_readfirstlane(w);
    const bool dk = wu < 4;
    const int hh = (wu >> 1) & 1, r8 = lane >> 3;
    const uint32_t kstep = dk ? FA_KT * 128u : FA_KT * 2u;
    uint32_t voff[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {  // lane: LDS row rowb, slot lane & 7, which holds chunk (lane & 7) ^ ((rowb >> 1) & 7)
        const int rowb = 8 * ((wu * 4 + i) & 7) + r8, ch = (lane & 7) ^ ((rowb >> 1) & 7);
        voff[i] = dk ? (uint32_t)((hh * TP + rowb) * 128 + ch * 16) : (uint32_t)((hh * XT_HD + rowb) * TP * 2 + ch * 16);
    }
    auto issue = [&](uint8_t *st, int kt) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(dk ? rk : rv, (lds_void *)(st + 1024 * (wu * 4 + i)), 16, voff[i],
                                                     (uint32_t)kt * kstep, 0, 0);
    };

    // Q fragments (B operand of S^T): query q0 + l32, dims 16 step + 8 g .. + 8
    v8bf qf[4];
    {
        const int qrow = active ? q0 + l32 : 0;
        const uint16_t *qp = q + ((size_t)b * XT_NH + head) * TP * XT_HD + (size_t)qrow * XT_HD + 8 * g;
#pragma unroll
        for (int s = 0; s < 4; s++) qf[s] = __builtin_bit_cast(v8bf, *(const uint4 *)(qp + 16 * s));
    }
    const int jrow = 16 * ((l32 >> 3) >> 1) + 8 * ((l32 >> 2) & 1) + 4 * ((l32 >> 3) & 1) + (l32 & 3);  // pi(l32)

    // bit 16 u + e: the key of accumulator e of 32-key half u in the last tile lies below T
    uint32_t kvalid = 0;
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int j = e >> 2, i = e & 3;
            const int key = (nkt - 1) * FA_KT + 32 * u + 16 * (j >> 1) + 8 * g + 4 * (j & 1) + i;
            kvalid |= (key < T ? 1u : 0u) << (16 * u + e);
        }

    v16f o[2];
    o[0] = v16f{};
    o[1] = v16f{};
    float mrun = -INFINITY, lsum = 0.f;

    // scores of one 64-key tile relative to the offset off (the accumulators start from -off), padded keys -inf
    auto scores = [&](const uint8_t *tk, int kt, float off, v16f (&s)[2]) {
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int e = 0; e < 16; e++) s[u][e] = -off;
        // the two 32-key halves' chains interleaved, each K fragment read one matrix instruction ahead of its use
        v8bf kf[2] = {frag_bf(tk, jrow, g), frag_bf(tk, 32 + jrow, g)};
#pragma unroll
        for (int step = 0; step < 4; step++)
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const v8bf f = kf[u];
                if (step + 1 < 4) kf[u] = frag_bf(tk, 32 * u + jrow, 2 * (step + 1) + g);
                s[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f, qf[step], s[u], 0, 0, 0);
            }
        if (!xkey && kt == nkt - 1 && (T & (FA_KT - 1))) {  // keys past T are padding
            uint32_t vm = kvalid;
            asm volatile("" : "+v"(vm));  // tested here, not as 32 lane masks held in scalar registers
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int e = 0; e < 16; e++)
                    if (!((vm >> (16 * u + e)) & 1u)) s[u][e] = -INFINITY;
        }
    };
    // the query's maximum over the tile (both lane halves)
    auto tile_max = [&](const v16f (&s)[2]) {
        float m0 = s[0][0], m1 = s[0][1], m2 = s[1][0], m3 = s[1][1];  // four chains, not one of 16
#pragma unroll
        for (int e = 2; e < 16; e += 2) {
            m0 = __builtin_fmaxf(m0, s[0][e]);
            m1 = __builtin_fmaxf(m1, s[0][e + 1]);
            m2 = __builtin_fmaxf(m2, s[1][e]);
            m3 = __builtin_fmaxf(m3, s[1][e + 1]);
        }
        const float t = __builtin_fmaxf(__builtin_fmaxf(m0, m1), __builtin_fmaxf(m2, m3));
        return __builtin_fmaxf(t, __shfl_xor(t, 32, 64));
    };
    // p = exp2(s) as the bf16 B operands of the PV product, and the sum of those bf16 values (two per v_dot2c)
    auto weights = [&](v16f (&s)[2], v8bf (&pf)[4]) {
        float t[2] = {0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int e = 0; e < 16; e++) s[u][e] = __builtin_amdgcn_exp2f(s[u][e]);
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int sp = 0; sp < 2; sp++) {
                const v8bf f = pack_p(s[u], 8 * sp);
                pf[2 * u + sp] = f;
                t[u] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(f, f, 0, 1), kOnes2, t[u], false);
                t[u] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(f, f, 2, 3), kOnes2, t[u], false);
                t[u] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(f, f, 4, 5), kOnes2, t[u], false);
                t[u] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(f, f, 6, 7), kOnes2, t[u], false);
            }
        return t[0] + t[1];
    };

    // one key tile on a resident stage. Each query's scores are taken relative to an offset mrun: the first tile
    // sets it to the query's maximum over that tile, and it is raised only when a later tile's weights would pass
    // 2^FA_PLOG (their bf16 sum, per lane, is the test), so no tile spends instructions on a running maximum
    auto tile = [&](const uint8_t *st, int kt) {
        const uint8_t *tk = st + hsel * FA_TILE, *tv = st + (2 + hsel) * FA_TILE;
        v16f s[2];
        v8bf pf[4];
        float tl;
        // at most two passes: the first tile's one pass sets the offset (key 0 is never padding, so its maximum is
        // finite); a later tile takes a second pass, with the offset raised to its maximum, only if a weight passed
        // the bound in the first
        bool fix = kt == 0;
        float off = kt == 0 ? 0.f : mrun;
        for (;;) {
            scores(tk, kt, off, s);
            if (fix) {
                const float tm = tile_max(s), mnew = kt == 0 ? tm : __builtin_fmaxf(tm, 0.f);
                if (kt != 0) {
                    const float sc = __builtin_amdgcn_exp2f(-mnew);
                    lsum *= sc;
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        o[0][e] *= sc;
                        o[1][e] *= sc;
                    }
                }
#pragma unroll
                for (int u = 0; u < 2; u++)
#pragma unroll
                    for (int e = 0; e < 16; e++) s[u][e] -= mnew;
                mrun = off + mnew;
            }
            tl = weights(s, pf);
            if (fix || __builtin_amdgcn_ballot_w64(!(tl <= FA_PMAX)) == 0) break;  // wave-uniform
            fix = true;
            off = mrun;
        }
        lsum += tl;
        // O^T += V^T P^T over the tile's four 16-key groups
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int sp = 0; sp < 2; sp++)
#pragma unroll
                for (int dt = 0; dt < 2; dt++)
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_bf(tv, 32 * dt + l32, 4 * u + 2 * sp + g),
                                                                   pf[2 * u + sp], o[dt], 0, 0, 0);
    };

    // two stages, the loop unrolled by two so each half's stage (and every LDS address in it) is fixed
    uint8_t *const st0 = smem, *const st1 = smem + FA_STAGE;
    if (nkt > 0) issue(st0, 0);
    for (int kt = 0; kt < nkt; kt += 2) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (kt + 1 < nkt) issue(st1, kt + 1);
        if (active) tile(st0, kt);
        if (kt + 1 >= nkt) break;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (kt + 2 < nkt) issue(st0, kt + 2);
        if (active) tile(st1, kt + 1);
    }

    if (xkey && active) {  // key T - 1: score from global memory, the same offset test, one bf16 weight
        const int kx = T - 1;
        const size_t hrow = ((size_t)b * XT_NH + head) * TP * XT_HD;
        const uint16_t *kr = k + hrow + (size_t)kx * XT_HD + 8 * g;
        float sx = 0.f;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const v8bf kk = __builtin_bit_cast(v8bf, *(const uint4 *)(kr + 16 * s));
            sx = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(qf[s], qf[s], 0, 1),
                                                 __builtin_shufflevector(kk, kk, 0, 1), sx, false);
            sx = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(qf[s], qf[s], 2, 3),
                                                 __builtin_shufflevector(kk, kk, 2, 3), sx, false);
            sx = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(qf[s], qf[s], 4, 5),
                                                 __builtin_shufflevector(kk, kk, 4, 5), sx, false);
            sx = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(qf[s], qf[s], 6, 7),
                                                 __builtin_shufflevector(kk, kk, 6, 7), sx, false);
        }
        sx += __shfl_xor(sx, 32, 64);
        float rel = sx - mrun;  // mrun is finite: at least one tile ran
        if (__builtin_amdgcn_ballot_w64(rel > FA_PLOG) != 0) {
            const float mnew = __builtin_fmaxf(0.f, rel), sc = __builtin_amdgcn_exp2f(-mnew);
            lsum *= sc;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                o[0][e] *= sc;
                o[1][e] *= sc;
            }
            rel -= mnew;
            mrun += mnew;
        }
        const __bf16 pb = (__bf16)__builtin_amdgcn_exp2f(rel);
        const float p = (float)pb;
        lsum += g == 0 ? p : 0.f;  // one lane of each query pair counts it: the halves are summed below
        const uint16_t *vr = vt + hrow + (size_t)kx;
#pragma unroll
        for (int dt = 0; dt < 2; dt++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int d = 32 * dt + 8 * (e >> 2) + 4 * g + (e & 3);
                o[dt][e] = __builtin_fmaf(p, __builtin_bit_cast(float, (uint32_t)vr[(size_t)d * TP] << 16), o[dt][e]);
            }
    }

    // normalise, then E4M3 with one scale per (query, 128 columns = this head pair)
    float amax = 0.f, inv_l = 0.f;
    if (active) {
        lsum += __shfl_xor(lsum, 32, 64);
        inv_l = 1.0f / lsum;
#pragma unroll
        for (int dt = 0; dt < 2; dt++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                o[dt][e] *= inv_l;
                amax = __builtin_fmaxf(amax, __builtin_fabsf(o[dt][e]));
            }
        amax = __builtin_fmaxf(amax, __shfl_xor(amax, 32, 64));
    }
    if (lane < 32) xamax[w * 32 + lane] = amax;
    __syncthreads();
    if (!active) return;
    amax = __builtin_fmaxf(amax, xamax[(w ^ 4) * 32 + l32]);
    const float sc = block_scale(amax), inv = block_scale_inv(sc);
    const int query = q0 + l32;
    if (query >= T) return;
    const size_t m = (size_t)b * T + query;
    uint8_t *dst = o8 + m * XT_D + head * XT_HD;
#pragma unroll
    for (int dt = 0; dt < 2; dt++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int d = 32 * dt + 8 * j + 4 * g;
            *(uint32_t *)(dst + d) = e4_pack4_scaled(o[dt][4 * j] * inv, o[dt][4 * j + 1] * inv,
                                                     o[dt][4 * j + 2] * inv, o[dt][4 * j + 3] * inv);
            if (DBG) {
                float *dd = o32 + m * XT_D + head * XT_HD + d;
                *(float4 *)dd = make_float4(o[dt][4 * j], o[dt][4 * j + 1], o[dt][4 * j + 2], o[dt][4 * j + 3]);
            }
        }
    if (hsel == 0 && g == 0) os[(size_t)hp * lds + m] = sc;
}

static int flash_launch(const char *what, const void *q, const void *k, const void *vt, void *o8, float *os, int lds,
                        int nseq, int T, int TP, float *o32, void *stream)
{
    if (nseq <= 0 || T <= 0 || TP < (T + FA_KT - 1) / FA_KT * FA_KT || lds < nseq * T || (size_t)2 * TP * XT_HD * 2 > 0xFFFFFFFFu)
        return xt_fail(what, "bad shape (nseq, T > 0; TP >= T rounded up to 64; lds >= nseq * T)");
    if ((((uintptr_t)q) | ((uintptr_t)k) | ((uintptr_t)vt) | ((uintptr_t)o8)) & 15)
        return xt_fail(what, "q, k, vt, o8 must be 16-byte aligned");
    static_assert(XT_NH / 2 == 8, "the XCD-aware block order groups 8 head pairs per sequence");
    if ((size_t)(T + FA_QB - 1) / FA_QB * (XT_NH / 2) * nseq > 0x7fffffffu) return xt_fail(what, "grid too large");
    const dim3 grid((T + FA_QB - 1) / FA_QB * (XT_NH / 2) * nseq);
    if (o32)
        hipLaunchKernelGGL(k_flash<1>, grid, dim3(512), 0, (hipStream_t)stream, (const uint16_t *)q, (const uint16_t *)k,
                           (const uint16_t *)vt, (uint8_t *)o8, os, lds, o32, T, TP);
    else
        hipLaunchKernelGGL(k_flash<0>, grid, dim3(512), 0, (hipStream_t)stream, (const uint16_t *)q, (const uint16_t *)k,
                           (const uint16_t *)vt, (uint8_t *)o8, os, lds, o32, T, TP);
    return xt_check(what);
}

extern "C" int eva_k_flash(const void *q, const void *k, const void *vt, void *o8, float *os, int lds, int nb,
                           float *o32, void *stream)
{
    return flash_launch("eva_k_flash", q, k, vt, o8, os, lds, nb, XT_T, XT_TP, o32, stream);
}

extern "C" int eva_k_flash_seq(const void *q, const void *k, const void *vt, void *o8, float *os, int lds, int nseq,
                               int T, int TP, float *o32, void *stream)
{
    return flash_launch("eva_k_flash_seq", q, k, vt, o8, os, lds, nseq, T, TP, o32, stream);
}
