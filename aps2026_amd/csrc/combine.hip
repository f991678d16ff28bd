// Weighted combine / unpermute, and the weight-packing kernels used at
// registration.
//
// Reference: k_moe_combine (src/tensor.cu:1968-1988) computes
// out[t][d] = 0 + 0.5*y[p_lo][d] + 0.5*y[p_hi][d].  0.5*v is exact in binary
// floating point, so the sum rounds once and its order cannot change a bit:
// RN(0.5a + 0.5b) is what every order gives.  Here one thread moves 8
// consecutive elements of one token (16-byte bf16 or 2x16-byte f32 loads),
// so every wave reads and writes whole 128-byte lines.
#include "common.hpp"

namespace aps {
namespace {

__device__ inline float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ inline uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

template <bool YBF16>
__device__ inline void load8(const void* y, int64_t off, float v[8]) {
    if (YBF16) {
        const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const bf16_t*>(y) + off);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = bf16_to_f32(w[i] & 0xffffu);
            v[2 * i + 1] = bf16_to_f32(w[i] >> 16);
        }
    } else {
        const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(y) + off);
        const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(y) + off + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
}

template <bool YBF16, bool OBF16>
__global__ void __launch_bounds__(256)
k_combine(const void* __restrict__ y, const uint32_t* __restrict__ route_positions, int64_t rows,
          int H, void* __restrict__ out) {
    const int per_row = H / 8;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= rows * per_row) return;
    const int64_t t = i / per_row;
    const int c = static_cast<int>(i - t * per_row) * 8;
    const uint32_t p0 = route_positions[2 * t];
    const uint32_t p1 = route_positions[2 * t + 1];
    float a[8], b[8], o[8];
    load8<YBF16>(y, static_cast<int64_t>(p0) * H + c, a);
    load8<YBF16>(y, static_cast<int64_t>(p1) * H + c, b);
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = __fadd_rn(__fmul_rn(0.5f, a[k]), __fmul_rn(0.5f, b[k]));
    if (OBF16) {
        uint4 q;
        q.x = f32_to_bf16_bits(o[0]) | (f32_to_bf16_bits(o[1]) << 16);
        q.y = f32_to_bf16_bits(o[2]) | (f32_to_bf16_bits(o[3]) << 16);
        q.z = f32_to_bf16_bits(o[4]) | (f32_to_bf16_bits(o[5]) << 16);
        q.w = f32_to_bf16_bits(o[6]) | (f32_to_bf16_bits(o[7]) << 16);
        *reinterpret_cast<uint4*>(static_cast<bf16_t*>(out) + t * H + c) = q;
    } else {
        float* d = static_cast<float*>(out) + t * H + c;
        *reinterpret_cast<float4*>(d) = make_float4(o[0], o[1], o[2], o[3]);
        *reinterpret_cast<float4*>(d + 4) = make_float4(o[4], o[5], o[6], o[7]);
    }
}

// Copies `nrows` rows of length H into the packed gate||up slab layout
// [F/64][128][H]: source row r goes to slab r/64, row (half*64 + r%64).
template <bool SRC_BF16>
__global__ void k_pack_rows_bf16(const void* __restrict__ src, bf16_t* __restrict__ dst, int nrows,
                                 int H, int half) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= static_cast<int64_t>(nrows) * H) return;
    const int r = static_cast<int>(i / H);
    const int k = static_cast<int>(i - static_cast<int64_t>(r) * H);
    const int64_t drow = static_cast<int64_t>(r / 64) * 128 + half * 64 + (r % 64);
    uint32_t v;
    if (SRC_BF16) v = static_cast<const bf16_t*>(src)[i];
    else v = f32_to_bf16_bits(static_cast<const float*>(src)[i]);
    dst[drow * H + k] = static_cast<bf16_t>(v);
}

__global__ void k_convert_bf16(const float* __restrict__ src, bf16_t* __restrict__ dst, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) dst[i] = static_cast<bf16_t>(f32_to_bf16_bits(src[i]));
}

}  // namespace

hipError_t launch_combine(const void* y, bool y_bf16, const uint32_t* route_positions,
                          int64_t rows, int hidden, void* out, bool out_bf16, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hidden % 8 != 0) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(ceil_div(rows * (hidden / 8), 256)));
    if (y_bf16 && out_bf16)
        hipLaunchKernelGGL((k_combine<true, true>), grid, dim3(256), 0, s, y, route_positions, rows, hidden, out);
    else if (y_bf16)
        hipLaunchKernelGGL((k_combine<true, false>), grid, dim3(256), 0, s, y, route_positions, rows, hidden, out);
    else if (out_bf16)
        hipLaunchKernelGGL((k_combine<false, true>), grid, dim3(256), 0, s, y, route_positions, rows, hidden, out);
    else
        hipLaunchKernelGGL((k_combine<false, false>), grid, dim3(256), 0, s, y, route_positions, rows, hidden, out);
    return hipGetLastError();
}

hipError_t launch_pack_w13_bf16(const void* const* w1, const void* const* w3, bool src_bf16,
                                bf16_t* dst, int experts, int ffn, int hidden, hipStream_t s) {
    const int64_t n = static_cast<int64_t>(ffn) * hidden;
    const dim3 grid(static_cast<unsigned>(ceil_div(n, 256)));
    for (int e = 0; e < experts; ++e) {
        bf16_t* d = dst + static_cast<int64_t>(e) * 2 * n;
        for (int half = 0; half < 2; ++half) {
            const void* src = half ? w3[e] : w1[e];
            if (src_bf16)
                hipLaunchKernelGGL(k_pack_rows_bf16<true>, grid, dim3(256), 0, s, src, d, ffn, hidden, half);
            else
                hipLaunchKernelGGL(k_pack_rows_bf16<false>, grid, dim3(256), 0, s, src, d, ffn, hidden, half);
        }
    }
    return hipGetLastError();
}

hipError_t launch_convert_to_bf16(const float* src, bf16_t* dst, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_convert_bf16, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0,
                       s, src, dst, n);
    return hipGetLastError();
}

}  // namespace aps
