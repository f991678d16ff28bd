// Measurement helper for bench.py (not part of the MoE library): the cost of
// the fp32 FMA chains that bound the router GEMM, measured on the device the
// bench runs on.
//
// aps_probe_fma_chain(waves_per_simd, dpp, chains, steps, cycles, clock_mhz)
// launches one workgroup of 4 * waves_per_simd waves per CU (waves_per_simd
// waves on each SIMD).  Every lane runs `chains` interleaved fp32 FMA chains
// of `steps` steps each (chains = 1: every FMA depends on the previous one;
// chains = 2: two independent accumulators alternate), as v_fmac_f32 or, with
// dpp != 0, v_fmac_f32_dpp with a row_newbcast operand (the router's
// instruction).  Each wave reads the shader clock (s_memtime) and the 100 MHz
// real-time counter (s_memrealtime) around its chain.  Results:
//   *cycles     shader-clock cycles per FMA instruction of one wave, averaged
//               over all waves;
//   *clock_mhz  the shader clock during the run, from the two counters.
// Returns 0, or a HIP error code.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace {

#define APS_PF(A, X, G) "v_fmac_f32 %" #A ", %" #X ", %" #G "\n\t"
#define APS_PD(A, X, G, L) "v_fmac_f32_dpp %" #A ", %" #X ", %" #G " row_newbcast:" #L " row_mask:0xf bank_mask:0xf\n\t"

// 16 FMA instructions per asm block; operands %0, %1 accumulators, %2..%9 x,
// %10..%17 g.  The x operands are written once, long before the first DPP
// read (a DPP source written by VALU needs two wait states).
template <bool DPP, int CHAINS>
__device__ inline void block16(float& a0, float& a1, const float (&x)[8], const float (&g)[8]) {
    if constexpr (!DPP && CHAINS == 1) {
        asm volatile(APS_PF(0, 2, 10) APS_PF(0, 3, 11) APS_PF(0, 4, 12) APS_PF(0, 5, 13) APS_PF(0, 6, 14)
                     APS_PF(0, 7, 15) APS_PF(0, 8, 16) APS_PF(0, 9, 17) APS_PF(0, 2, 10) APS_PF(0, 3, 11)
                     APS_PF(0, 4, 12) APS_PF(0, 5, 13) APS_PF(0, 6, 14) APS_PF(0, 7, 15) APS_PF(0, 8, 16)
                     APS_PF(0, 9, 17)
                     : "+v"(a0), "+v"(a1)
                     : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]), "v"(x[6]), "v"(x[7]),
                       "v"(g[0]), "v"(g[1]), "v"(g[2]), "v"(g[3]), "v"(g[4]), "v"(g[5]), "v"(g[6]), "v"(g[7]));
    } else if constexpr (!DPP) {
        asm volatile(APS_PF(0, 2, 10) APS_PF(1, 3, 11) APS_PF(0, 4, 12) APS_PF(1, 5, 13) APS_PF(0, 6, 14)
                     APS_PF(1, 7, 15) APS_PF(0, 8, 16) APS_PF(1, 9, 17) APS_PF(0, 2, 10) APS_PF(1, 3, 11)
                     APS_PF(0, 4, 12) APS_PF(1, 5, 13) APS_PF(0, 6, 14) APS_PF(1, 7, 15) APS_PF(0, 8, 16)
                     APS_PF(1, 9, 17)
                     : "+v"(a0), "+v"(a1)
                     : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]), "v"(x[6]), "v"(x[7]),
                       "v"(g[0]), "v"(g[1]), "v"(g[2]), "v"(g[3]), "v"(g[4]), "v"(g[5]), "v"(g[6]), "v"(g[7]));
    } else if constexpr (CHAINS == 1) {
        asm volatile(APS_PD(0, 2, 10, 0) APS_PD(0, 3, 11, 0) APS_PD(0, 4, 12, 0) APS_PD(0, 5, 13, 0)
                     APS_PD(0, 6, 14, 0) APS_PD(0, 7, 15, 0) APS_PD(0, 8, 16, 0) APS_PD(0, 9, 17, 0)
                     APS_PD(0, 2, 10, 1) APS_PD(0, 3, 11, 1) APS_PD(0, 4, 12, 1) APS_PD(0, 5, 13, 1)
                     APS_PD(0, 6, 14, 1) APS_PD(0, 7, 15, 1) APS_PD(0, 8, 16, 1) APS_PD(0, 9, 17, 1)
                     : "+v"(a0), "+v"(a1)
                     : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]), "v"(x[6]), "v"(x[7]),
                       "v"(g[0]), "v"(g[1]), "v"(g[2]), "v"(g[3]), "v"(g[4]), "v"(g[5]), "v"(g[6]), "v"(g[7]));
    } else {
        asm volatile(APS_PD(0, 2, 10, 0) APS_PD(1, 3, 11, 0) APS_PD(0, 4, 12, 0) APS_PD(1, 5, 13, 0)
                     APS_PD(0, 6, 14, 0) APS_PD(1, 7, 15, 0) APS_PD(0, 8, 16, 0) APS_PD(1, 9, 17, 0)
                     APS_PD(0, 2, 10, 1) APS_PD(1, 3, 11, 1) APS_PD(0, 4, 12, 1) APS_PD(1, 5, 13, 1)
                     APS_PD(0, 6, 14, 1) APS_PD(1, 7, 15, 1) APS_PD(0, 8, 16, 1) APS_PD(1, 9, 17, 1)
                     : "+v"(a0), "+v"(a1)
                     : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]), "v"(x[6]), "v"(x[7]),
                       "v"(g[0]), "v"(g[1]), "v"(g[2]), "v"(g[3]), "v"(g[4]), "v"(g[5]), "v"(g[6]), "v"(g[7]));
    }
}

// times[2 w] = shader-clock cycles, times[2 w + 1] = 100 MHz ticks of wave w
template <bool DPP, int CHAINS>
__global__ void __launch_bounds__(1024) k_fma_chain(int blocks, float* __restrict__ sink,
                                                    long long* __restrict__ times) {
    const int lane = threadIdx.x & 63;
    float x[8], g[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        x[i] = 1.0f + 0x1p-20f * static_cast<float>(lane + i);
        g[i] = 0.5f - 0x1p-21f * static_cast<float>(i);
    }
    float a0 = 0.0f, a1 = 1.0f;
    const long long c0 = __builtin_readcyclecounter();
    const long long r0 = __builtin_amdgcn_s_memrealtime();
    for (int b = 0; b < blocks; ++b) block16<DPP, CHAINS>(a0, a1, x, g);
    const long long c1 = __builtin_readcyclecounter();
    const long long r1 = __builtin_amdgcn_s_memrealtime();
    const int w = blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
    sink[blockIdx.x * blockDim.x + threadIdx.x] = a0 + a1;
    if (lane == 0) {
        times[2 * w] = c1 - c0;
        times[2 * w + 1] = r1 - r0;
    }
}

}  // namespace

extern "C" __attribute__((visibility("default"))) int aps_probe_fma_chain(int waves_per_simd, int dpp, int chains,
                                                                        int steps, double* cycles,
                                                                        double* clock_mhz) {
    if (waves_per_simd < 1 || waves_per_simd > 4 || (chains != 1 && chains != 2) || steps < 16 || !cycles ||
        !clock_mhz)
        return static_cast<int>(hipErrorInvalidValue);
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return static_cast<int>(e);
    const int threads = 256 * waves_per_simd;
    const int waves = cus * threads / 64;
    float* sink = nullptr;
    long long* times = nullptr;
    if ((e = hipMalloc(&sink, sizeof(float) * cus * threads)) != hipSuccess) return static_cast<int>(e);
    if ((e = hipMalloc(&times, sizeof(long long) * 2 * waves)) != hipSuccess) {
        (void)hipFree(sink);
        return static_cast<int>(e);
    }
    auto kern = dpp ? (chains == 1 ? k_fma_chain<true, 1> : k_fma_chain<true, 2>)
                    : (chains == 1 ? k_fma_chain<false, 1> : k_fma_chain<false, 2>);
    const int blocks = steps / 16;
    std::vector<long long> h(2 * static_cast<size_t>(waves));
    for (int rep = 0; rep < 3 && e == hipSuccess; ++rep) {  // the last of three runs is kept
        hipLaunchKernelGGL(kern, dim3(cus), dim3(threads), 0, 0, blocks, sink, times);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipDeviceSynchronize();
    }
    if (e == hipSuccess) e = hipMemcpy(h.data(), times, h.size() * sizeof(long long), hipMemcpyDeviceToHost);
    (void)hipFree(sink);
    (void)hipFree(times);
    if (e != hipSuccess) return static_cast<int>(e);
    double cyc = 0.0, rt = 0.0;
    for (int w = 0; w < waves; ++w) {
        cyc += static_cast<double>(h[2 * w]);
        rt += static_cast<double>(h[2 * w + 1]);
    }
    *cycles = cyc / waves / (16.0 * blocks);
    *clock_mhz = rt > 0.0 ? cyc / rt * 100.0 : 0.0;
    return 0;
}
