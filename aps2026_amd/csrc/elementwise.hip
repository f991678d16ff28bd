// Elementwise fp32 ops of the decoder layer and the dense MLP.
//
// Reference kernels (src/tensor.cu:1990-2010) and launchers (:3236-3260,
// zero_gpu :277-281):
//   k_add       a[i] += b[i]
//   k_add_bias  a[i] += bias[i % h]
//   k_silu_mul  out[i] = (g / (1 + (float)exp((double)-g))) * up[i]
//   zero_gpu    x[i] = 0
// Each element is one rounded fp32 operation (two for SiLU-mul, with the
// division correctly rounded), so the results equal the reference's bit for
// bit.  gfx950 mapping: a thread owns four consecutive elements and moves
// them as one 16-byte access when the arrays are 16-byte aligned and the
// count is a multiple of four; a scalar kernel covers the rest.  Zero is a
// kernel, not hipMemsetAsync, so a caller may record it into a HIP graph.
#include "common.hpp"

namespace aps {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

__device__ inline float silu_mul_ref(float g, float u) {
    const float e = static_cast<float>(exp(-static_cast<double>(g)));
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, e)), u);
}

__global__ void __launch_bounds__(256) k_add4(v4f* __restrict__ a, const v4f* __restrict__ b, int64_t n4) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n4) return;
    v4f x = a[i];
    const v4f y = b[i];
    x[0] = __fadd_rn(x[0], y[0]);
    x[1] = __fadd_rn(x[1], y[1]);
    x[2] = __fadd_rn(x[2], y[2]);
    x[3] = __fadd_rn(x[3], y[3]);
    a[i] = x;
}

__global__ void __launch_bounds__(256) k_add1(float* __restrict__ a, const float* __restrict__ b, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) a[i] = __fadd_rn(a[i], b[i]);
}

// h % 4 == 0 here, so a 4-element group never straddles a row
__global__ void __launch_bounds__(256) k_add_bias4(v4f* __restrict__ a, const float* __restrict__ bias, int64_t n4,
                                                   int h4) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n4) return;
    const v4f bv = reinterpret_cast<const v4f*>(bias)[i % h4];
    v4f x = a[i];
    x[0] = __fadd_rn(x[0], bv[0]);
    x[1] = __fadd_rn(x[1], bv[1]);
    x[2] = __fadd_rn(x[2], bv[2]);
    x[3] = __fadd_rn(x[3], bv[3]);
    a[i] = x;
}

__global__ void __launch_bounds__(256) k_add_bias1(float* __restrict__ a, const float* __restrict__ bias, int64_t n,
                                                   int h) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) a[i] = __fadd_rn(a[i], bias[i % h]);
}

__global__ void __launch_bounds__(256) k_silu_mul4(const v4f* __restrict__ g, const v4f* __restrict__ u,
                                                   v4f* __restrict__ out, int64_t n4) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n4) return;
    const v4f gv = g[i], uv = u[i];
    v4f o;
    o[0] = silu_mul_ref(gv[0], uv[0]);
    o[1] = silu_mul_ref(gv[1], uv[1]);
    o[2] = silu_mul_ref(gv[2], uv[2]);
    o[3] = silu_mul_ref(gv[3], uv[3]);
    out[i] = o;
}

__global__ void __launch_bounds__(256) k_silu_mul1(const float* __restrict__ g, const float* __restrict__ u,
                                                   float* __restrict__ out, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) out[i] = silu_mul_ref(g[i], u[i]);
}

__global__ void __launch_bounds__(256) k_zero4(v4f* __restrict__ x, int64_t n4) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n4) x[i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
}

__global__ void __launch_bounds__(256) k_zero1(float* __restrict__ x, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) x[i] = 0.0f;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

dim3 grid_for(int64_t n) { return dim3(static_cast<unsigned>(ceil_div(n, 256))); }

}  // namespace

hipError_t launch_add_inplace(float* a, const float* b, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (n % 4 == 0 && aligned16(a) && aligned16(b))
        hipLaunchKernelGGL(k_add4, grid_for(n / 4), dim3(256), 0, s, reinterpret_cast<v4f*>(a),
                           reinterpret_cast<const v4f*>(b), n / 4);
    else
        hipLaunchKernelGGL(k_add1, grid_for(n), dim3(256), 0, s, a, b, n);
    return hipGetLastError();
}

hipError_t launch_add_bias(float* a, const float* bias, int64_t n, int h, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (h % 4 == 0 && n % 4 == 0 && aligned16(a) && aligned16(bias))
        hipLaunchKernelGGL(k_add_bias4, grid_for(n / 4), dim3(256), 0, s, reinterpret_cast<v4f*>(a), bias, n / 4,
                           h / 4);
    else
        hipLaunchKernelGGL(k_add_bias1, grid_for(n), dim3(256), 0, s, a, bias, n, h);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float* g, const float* u, float* out, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (n % 4 == 0 && aligned16(g) && aligned16(u) && aligned16(out))
        hipLaunchKernelGGL(k_silu_mul4, grid_for(n / 4), dim3(256), 0, s, reinterpret_cast<const v4f*>(g),
                           reinterpret_cast<const v4f*>(u), reinterpret_cast<v4f*>(out), n / 4);
    else
        hipLaunchKernelGGL(k_silu_mul1, grid_for(n), dim3(256), 0, s, g, u, out, n);
    return hipGetLastError();
}

hipError_t launch_zero(float* x, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (n % 4 == 0 && aligned16(x))
        hipLaunchKernelGGL(k_zero4, grid_for(n / 4), dim3(256), 0, s, reinterpret_cast<v4f*>(x), n / 4);
    else
        hipLaunchKernelGGL(k_zero1, grid_for(n), dim3(256), 0, s, x, n);
    return hipGetLastError();
}

}  // namespace aps
