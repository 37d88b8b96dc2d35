// peak.hip - on-box measurement of the ceilings the roofline fractions are taken against: dense FP8 MFMA
// throughput (v_mfma_f32_16x16x128_f8f6f4 on register operands), HBM stream-copy bandwidth, and LDS read bandwidth
// (ds_read_b128). No reference counterpart: the reference publishes no kernel-level numbers; these entry points exist
// so every fraction reported beside a benchmark uses a peak measured on the same GPU.
#include "xt_abi.h"
#include "xt_common.h"
#include "gemm_core.h"

// Each wave keeps 8 independent accumulator chains so back-to-back MFMAs never wait on each other.
__global__ void __launch_bounds__(256) k_peak_mfma(int iters, float *__restrict__ out)
{
    const int lane = threadIdx.x & 63;
    v8i a, b;
    for (int i = 0; i < 8; i++) {
        a[i] = 0x38383838 ^ (lane * 0x01010101 + i);   // finite E4M3 bytes, lane dependent
        b[i] = 0x30303030 ^ (lane + i * 0x00010001);
    }
    v4f acc[8];
    for (int c = 0; c < 8; c++) acc[c] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int c = 0; c < 8; c++)
            acc[c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc[c], 0, 0, 0, 0, 0, 0);
    }
    float s = 0.f;
    for (int c = 0; c < 8; c++) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
    out[blockIdx.x * 256 + threadIdx.x] = s;
}

// Stream copy: block b moves the 4 KB at 4 KB * b, one 16-byte load and store per thread, both nontemporal. With a
// block per 4 KB the blocks in flight touch neighbouring DRAM pages: 6.2-6.5 TB/s on MI355X over 1 GiB, where a
// grid-stride loop (each wave's loads tens of MB apart) reached 5.2 and torch's device copy 5.0.
typedef unsigned peak_v4u __attribute__((ext_vector_type(4)));
__global__ void __launch_bounds__(256) k_peak_copy(const peak_v4u *__restrict__ src, peak_v4u *__restrict__ dst,
                                                   long n16)
{
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i < n16) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// 256 threads issue 16 ds_read_b128 per iteration (lane-linear 1 KB rows, conflict-free) from inline assembly, so no
// ALU work consumes the data and the loop is bound by the LDS read path alone.
__global__ void __launch_bounds__(256) k_peak_lds(int iters, uint32_t *__restrict__ out)
{
    __shared__ __attribute__((aligned(16))) uint4 buf[4096];
    for (int i = threadIdx.x; i < 4096; i += 256) buf[i] = make_uint4(i, i * 3, i * 5, i * 7);
    __syncthreads();
    const uint32_t a = lds_addr(buf) + (uint32_t)((threadIdx.x >> 6) * 4096 + (threadIdx.x & 63) * 16);  // + 15 KB < 64 KB
    v4i v0, v1;
    for (int it = 0; it < iters; it++) {
#define XT_RD2(o0, o1) asm volatile("ds_read_b128 %0, %2 offset:" #o0 "\n\tds_read_b128 %1, %2 offset:" #o1 \
                                    : "=v"(v0), "=v"(v1) : "v"(a));
        XT_RD2(0, 1024) XT_RD2(2048, 3072) XT_RD2(4096, 5120) XT_RD2(6144, 7168)
        XT_RD2(8192, 9216) XT_RD2(10240, 11264) XT_RD2(12288, 13312) XT_RD2(14336, 15360)
#undef XT_RD2
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    out[blockIdx.x * 256 + threadIdx.x] = (uint32_t)(v0[0] ^ v1[3]);
}

extern "C" int eva_probe_mfma_fp8(int blocks, int iters, float *out, void *stream)
{
    if (blocks <= 0 || iters <= 0) return xt_fail("eva_probe_mfma_fp8", "blocks and iters must be positive");
    hipLaunchKernelGGL(k_peak_mfma, dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters, out);
    return xt_check("eva_probe_mfma_fp8");
}

extern "C" int eva_probe_copy(const void *src, void *dst, size_t bytes, void *stream)
{
    if (bytes % 16 || (((uintptr_t)src | (uintptr_t)dst) & 15)) return xt_fail("eva_probe_copy", "16-byte multiples");
    const long n16 = (long)(bytes / 16), blocks = (n16 + 255) / 256;
    if (blocks > 0x7fffffffL) return xt_fail("eva_probe_copy", "at most 2^31 - 1 blocks of 4 KB");
    if (blocks == 0) return 0;
    hipLaunchKernelGGL(k_peak_copy, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (const peak_v4u *)src,
                       (peak_v4u *)dst, n16);
    return xt_check("eva_probe_copy");
}

extern "C" int eva_probe_lds(int blocks, int iters, uint32_t *out, void *stream)
{
    if (blocks <= 0 || iters <= 0) return xt_fail("eva_probe_lds", "blocks and iters must be positive");
    hipLaunchKernelGGL(k_peak_lds, dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters, out);
    return xt_check("eva_probe_lds");
}
