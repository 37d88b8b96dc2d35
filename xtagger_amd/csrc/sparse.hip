// sparse.hip - 2:4 structured sparsity of the E4M3 block weights (the 2:4-sparse workload): magnitude pruning along K
// (the role of src/tools/prune24.py:43-56, "mag" rule) and packing into the compressed layout the sparse GEMM
// (gemm_core.h, bs_mainloop_sp) reads. The 128 x 128 block scales of the dense weights are kept unchanged.
#include "gemm_core.h"
#include "xt_abi.h"

// E4M3 magnitude order is code order: codes 0x00 .. 0x7E increase in value, so |dec(q)| compares as q & 0x7F.
// In each group of 4 consecutive k, the 2 lowest (|q|, k) in ascending order are zeroed: ties drop the lower k first.
__global__ void __launch_bounds__(256) k_prune24(uint8_t *__restrict__ w, long groups)
{
    for (long gi = (long)blockIdx.x * 256 + threadIdx.x; gi < groups; gi += (long)gridDim.x * 256) {
        uint32_t v = ((uint32_t *)w)[gi];
        int key[4];
#pragma unroll
        for (int i = 0; i < 4; i++) key[i] = (int)((v >> (8 * i)) & 0x7F) * 4 + i;  // (|q|, k) as one ordered key
        uint32_t keep = 0xFFFFFFFFu;
#pragma unroll
        for (int d = 0; d < 2; d++) {
            int lo = 0;
#pragma unroll
            for (int i = 1; i < 4; i++) lo = key[i] < key[lo] ? i : lo;
            keep &= ~(0xFFu << (8 * lo));
            key[lo] = 0x7FFFFFFF;
        }
        ((uint32_t *)w)[gi] = v & keep;
    }
}

// One thread per (16-row tile t, K block kb, lane l = 16 g + r): row 16 t + r, dense k [128 kb + 32 g, +32) -> 16
// value bytes and one index word (nibble j = p0 | p1 << 2). Kept positions: the nonzero bytes of each group of 4,
// completed with its lowest-k zero positions; a group with more than 2 nonzero bytes counts into *bad.
__global__ void __launch_bounds__(256) k_pack24(const uint8_t *__restrict__ w, int N, int K, uint8_t *__restrict__ vals,
                                                uint32_t *__restrict__ idx, int *__restrict__ bad)
{
    const int KB = K >> 7;
    const long items = (long)(N >> 4) * KB * 64;
    for (long it = (long)blockIdx.x * 256 + threadIdx.x; it < items; it += (long)gridDim.x * 256) {
        const int l = (int)(it & 63), g = l >> 4, r = l & 15;
        const long tk = it >> 6;
        const int t = (int)(tk / KB), kb = (int)(tk - (long)t * KB);
        const uint4 *src = (const uint4 *)(w + (size_t)(16 * t + r) * K + 128 * kb + 32 * g);
        const uint4 a = src[0], b = src[1];
        const uint32_t word[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t out[4] = {0, 0, 0, 0}, ix = 0;
        int nbad = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t v = word[j];
            int p0 = -1, p1 = -1, nz = 0;
#pragma unroll
            for (int i = 0; i < 4; i++)
                if ((v >> (8 * i)) & 0xFF) {
                    nz++;
                    if (p0 < 0) p0 = i;
                    else if (p1 < 0) p1 = i;
                }
            nbad += nz > 2;
#pragma unroll
            for (int i = 0; i < 4; i++)  // complete with the lowest-k zero positions
                if (!((v >> (8 * i)) & 0xFF)) {
                    if (p0 < 0) p0 = i;
                    else if (p1 < 0 && i != p0) p1 = i;
                }
            if (p0 > p1) { const int s = p0; p0 = p1; p1 = s; }
            const uint32_t two = ((v >> (8 * p0)) & 0xFF) | ((v >> (8 * p1)) & 0xFF) << 8;
            out[j >> 1] |= two << (16 * (j & 1));
            ix |= (uint32_t)(p0 | p1 << 2) << (4 * j);
        }
        *(uint4 *)(vals + it * 16) = make_uint4(out[0], out[1], out[2], out[3]);
        idx[it] = ix;
        if (nbad && bad) atomicAdd(bad, nbad);
    }
}

static int grid_of(long items)
{
    const long b = (items + 255) / 256;
    return (int)(b < 1 ? 1 : b > 65535 ? 65535 : b);
}

extern "C" int eva_k_prune24(void *w, int N, int K, void *stream)
{
    if (N <= 0 || K <= 0 || K % 4) return xt_fail("eva_k_prune24", "bad shape (N > 0, K > 0, K % 4 == 0)");
    if (((uintptr_t)w) & 3) return xt_fail("eva_k_prune24", "w must be 4-byte aligned");
    const long groups = (long)N * K / 4;
    hipLaunchKernelGGL(k_prune24, dim3(grid_of(groups)), dim3(256), 0, (hipStream_t)stream, (uint8_t *)w, groups);
    return xt_check("eva_k_prune24");
}

extern "C" int eva_k_pack24(const void *w, int N, int K, void *vals, void *idx, int *bad, void *stream)
{
    if (N <= 0 || N % 16 || K <= 0 || K % 128) return xt_fail("eva_k_pack24", "bad shape (N % 16 == 0, K % 128 == 0)");
    if ((((uintptr_t)w) | ((uintptr_t)vals)) & 15 || ((uintptr_t)idx) & 3)
        return xt_fail("eva_k_pack24", "w and vals must be 16-byte aligned, idx 4-byte aligned");
    const long items = (long)(N / 16) * (K / 128) * 64;
    hipLaunchKernelGGL(k_pack24, dim3(grid_of(items)), dim3(256), 0, (hipStream_t)stream, (const uint8_t *)w, N, K,
                       (uint8_t *)vals, (uint32_t *)idx, bad);
    return xt_check("eva_k_pack24");
}
