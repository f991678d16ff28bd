// Weighted combine / unpermute, and the weight-packing kernels used at
// registration.
//
// Reference: k_moe_combine (src/tensor.cu:1968-1988) computes
// out[t][d] = (0 + 0.5*y[p_lo][d]) + 0.5*y[p_hi][d].  0.5*v is exact in
// binary floating point, so the sum rounds once and the order of the two
// terms cannot change a bit; the leading 0 matters only for signed zeros
// (0 + -0 = +0, so two -0 terms give +0) and is kept (moe_combine2).  Here one
// thread moves 8 consecutive elements of one token (16-byte bf16 or
// 2x16-byte f32 loads), so every wave reads and writes whole 128-byte lines.
#include "common.hpp"

namespace aps {
namespace {

__device__ inline float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bits, round to nearest even (gfx950 v_cvt_pk_bf16_f32).
__device__ inline uint32_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ inline uint32_t pack2_bf16(float lo, float hi) {
    bf16x2_t v;
    v[0] = static_cast<__bf16>(lo);
    v[1] = static_cast<__bf16>(hi);
    return __builtin_bit_cast(uint32_t, v);
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
    for (int k = 0; k < 8; ++k) o[k] = moe_combine2(a[k], b[k]);
    if (OBF16) {
        uint4 q;
        q.x = pack2_bf16(o[0], o[1]);
        q.y = pack2_bf16(o[2], o[3]);
        q.z = pack2_bf16(o[4], o[5]);
        q.w = pack2_bf16(o[6], o[7]);
        *reinterpret_cast<uint4*>(static_cast<bf16_t*>(out) + t * H + c) = q;
    } else {
        float* d = static_cast<float*>(out) + t * H + c;
        *reinterpret_cast<float4*>(d) = make_float4(o[0], o[1], o[2], o[3]);
        *reinterpret_cast<float4*>(d + 4) = make_float4(o[4], o[5], o[6], o[7]);
    }
}

// Weight packing into MFMA tile images.  A B-operand stage of the grouped
// GEMMs is a 128-row x 64-k bf16 tile (16 KB).  Registration stores every
// such tile contiguously and already in the XOR-swizzled order the kernels
// keep in LDS (physical 16-byte chunk = chunk ^ ((row >> 1) & 7)), so one
// stage is one contiguous 16 KB block: the direct-to-LDS loads of a stage
// spread evenly over the L2 channels (a row-major weight would put every
// row of a stage 8 KB apart) and lane i simply copies bytes [16i, 16i+16)
// of each 1 KB slot.
//   w13: [E][F/64][H/64][128][64]  tile rows 0..63 = w1 rows nb*64 + r,
//                                  rows 64..127   = w3 rows nb*64 + r - 64
//   w2 : [E][H/128][F/64][128][64] tile rows = w2 rows nb*128 + r
// `split` is 64 for w13 (two sources) and 128 for w2 (one source).
template <bool SRC_BF16>
__global__ void k_pack_tiles(const void* __restrict__ src_lo, const void* __restrict__ src_hi,
                             bf16_t* __restrict__ dst, int K, int n_blocks, int split) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int KT = K / 64;
    const int64_t total = static_cast<int64_t>(n_blocks) * KT * 128 * 64;
    if (i >= total) return;
    const int pk = static_cast<int>(i & 63);
    const int r = static_cast<int>((i >> 6) & 127);
    const int64_t t = i >> 13;             // tile index = nb * KT + kt
    const int kt = static_cast<int>(t % KT);
    const int nb = static_cast<int>(t / KT);
    const int c = (pk >> 3) ^ ((r >> 1) & 7);
    const int k = kt * 64 + c * 8 + (pk & 7);
    const void* src = (split == 64 && r >= 64) ? src_hi : src_lo;
    const int64_t srow = static_cast<int64_t>(nb) * split + (r % split);
    uint32_t v;
    if (SRC_BF16) v = static_cast<const bf16_t*>(src)[srow * K + k];
    else v = f32_to_bf16_bits(static_cast<const float*>(src)[srow * K + k]);
    dst[i] = static_cast<bf16_t>(v);
}

// dst[i] = bf16(src[i]), round to nearest even; 8 elements per thread.
__global__ void __launch_bounds__(256)
k_to_bf16(const float* __restrict__ src, bf16_t* __restrict__ dst, int64_t n) {
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 8;
    if (i + 8 <= n) {
        const float4 a = *reinterpret_cast<const float4*>(src + i);
        const float4 b = *reinterpret_cast<const float4*>(src + i + 4);
        uint4 q;
        q.x = pack2_bf16(a.x, a.y);
        q.y = pack2_bf16(a.z, a.w);
        q.z = pack2_bf16(b.x, b.y);
        q.w = pack2_bf16(b.z, b.w);
        *reinterpret_cast<uint4*>(dst + i) = q;
    } else {
        for (int64_t j = i; j < n; ++j) dst[j] = static_cast<bf16_t>(f32_to_bf16_bits(src[j]));
    }
}

}  // namespace

hipError_t launch_to_bf16(const float* src, bf16_t* dst, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_to_bf16, dim3(static_cast<unsigned>(ceil_div(ceil_div(n, 8), 256))), dim3(256), 0, s,
                       src, dst, n);
    return hipGetLastError();
}

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
    const int64_t per_expert = static_cast<int64_t>(2) * ffn * hidden;
    const dim3 grid(static_cast<unsigned>(ceil_div(per_expert, 256)));
    for (int e = 0; e < experts; ++e) {
        bf16_t* d = dst + static_cast<int64_t>(e) * per_expert;
        if (src_bf16)
            hipLaunchKernelGGL(k_pack_tiles<true>, grid, dim3(256), 0, s, w1[e], w3[e], d, hidden, ffn / 64, 64);
        else
            hipLaunchKernelGGL(k_pack_tiles<false>, grid, dim3(256), 0, s, w1[e], w3[e], d, hidden, ffn / 64, 64);
    }
    return hipGetLastError();
}

hipError_t launch_pack_w2_bf16(const void* const* w2, bool src_bf16, bf16_t* dst, int experts, int ffn,
                               int hidden, hipStream_t s) {
    const int64_t per_expert = static_cast<int64_t>(ffn) * hidden;
    const dim3 grid(static_cast<unsigned>(ceil_div(per_expert, 256)));
    for (int e = 0; e < experts; ++e) {
        bf16_t* d = dst + static_cast<int64_t>(e) * per_expert;
        if (src_bf16)
            hipLaunchKernelGGL(k_pack_tiles<true>, grid, dim3(256), 0, s, w2[e], w2[e], d, ffn, hidden / 128, 128);
        else
            hipLaunchKernelGGL(k_pack_tiles<false>, grid, dim3(256), 0, s, w2[e], w2[e], d, ffn, hidden / 128, 128);
    }
    return hipGetLastError();
}

}  // namespace aps
