// fp8 e4m3 quantisation for the fp8 expert path, and its weight packing.
//
// The reference has no fp8 path; this is the library's own format (config
// C5, 8192 tokens with fp8 experts): weights e4m3 with one fp32 scale per output channel, x and the
// SwiGLU activations quantised per row at run time:
//   scale = amax(|row|) / 448 (1 if the row is all zero),
//   code  = e4m3(v / scale), round to nearest even, saturating at +-448
// (OCP "e4m3fn": bias 7, max 448, no infinities).  The quotient and the
// conversion below reproduce that definition bit for bit (IEEE division,
// then nearest-even e4m3), so the codes match the CPU oracle's encoder.
#include "common.hpp"

namespace aps {
namespace {

typedef e4m3_words_t u32x4_t;
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// The arithmetic (scale, quotient, code) is in common.hpp, shared with the
// router's x quantisation.

// One wave per row of n bf16 values (n % 8 == 0, n <= 512 * CH): each lane
// holds up to CH chunks of 8 values.  Writes n codes then zeros up to
// dst_stride (a multiple of 8), and the row's scale.
template <int CH>
__global__ void __launch_bounds__(64)
k_quant_rows(const bf16_t* __restrict__ src, int64_t src_stride, int n, uint8_t* __restrict__ dst,
             int64_t dst_stride, float* __restrict__ scale, int64_t rows) {
    const int64_t row = blockIdx.x;
    if (row >= rows) return;
    const int lane = threadIdx.x;
    const int nch = n / 8;
    const bf16_t* s = src + row * src_stride;
    u32x4_t v[CH];
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int ch = lane + 64 * c;
        v[c] = ch < nch ? *reinterpret_cast<const u32x4_t*>(s + ch * 8) : u32x4_t{0u, 0u, 0u, 0u};
        amax = e4m3_amax8(amax, v[c]);
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) amax = fmaxf(amax, __shfl_xor(amax, d));
    const float sc = e4m3_row_scale(amax);
    const float rc = __fdiv_rn(1.0f, sc);
    const bool fast = sc >= kMinFastScale;  // wave-uniform
    if (lane == 0) scale[row] = sc;
    uint8_t* d8 = dst + row * dst_stride;
    const int dch = static_cast<int>(dst_stride / 8);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int ch = lane + 64 * c;
        if (ch >= dch) continue;
        uint32_t lo = 0, hi = 0;
        if (ch < nch) {
            if (fast) e4m3_chunk_codes<true>(v[c], sc, rc, lo, hi);
            else e4m3_chunk_codes<false>(v[c], sc, rc, lo, hi);
        }
        *reinterpret_cast<u32x2_t*>(d8 + ch * 8) = u32x2_t{lo, hi};
    }
}

// fp8 weight tile images: 128 rows x 128 bytes (128 k) per image, 16-byte
// chunks swizzled as the MFMA kernels hold them in LDS (physical chunk =
// chunk ^ ((row >> 1) & 7)); k past K is zero.
//   w13: [E][F/64][H/128][128][128]  rows 0..63 = w1 rows nb*64 + r,
//                                    rows 64..127 = w3 rows nb*64 + r - 64
//   w2 : [E][H/128][Kp/128][128][128] rows = w2 rows nb*128 + r, Kp = F
//                                    rounded up to 128
// `split` is 64 for w13 (two sources) and 128 for w2.
__global__ void k_pack_tiles_e4m3(const uint8_t* __restrict__ src_lo, const uint8_t* __restrict__ src_hi,
                                  uint8_t* __restrict__ dst, int K, int KT, int n_blocks, int split) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t total = static_cast<int64_t>(n_blocks) * KT * 128 * 128;
    if (i >= total) return;
    const int pk = static_cast<int>(i & 127);
    const int r = static_cast<int>((i >> 7) & 127);
    const int64_t t = i >> 14;  // image index = nb * KT + kt
    const int kt = static_cast<int>(t % KT);
    const int nb = static_cast<int>(t / KT);
    const int c = (pk >> 4) ^ ((r >> 1) & 7);
    const int k = kt * 128 + c * 16 + (pk & 15);
    const uint8_t* src = (split == 64 && r >= 64) ? src_hi : src_lo;
    const int64_t srow = static_cast<int64_t>(nb) * split + (r % split);
    dst[i] = k < K ? src[srow * K + k] : static_cast<uint8_t>(0);
}

}  // namespace

hipError_t launch_quant_rows_e4m3(const bf16_t* src, int64_t src_stride, int n, uint8_t* dst, int64_t dst_stride,
                                  float* scale, int64_t rows, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (n % 8 != 0 || dst_stride % 8 != 0 || dst_stride < n) return hipErrorInvalidValue;
    const int chunks = static_cast<int>(ceil_div(dst_stride, 8));
    const dim3 grid(static_cast<unsigned>(rows));
    if (chunks <= 64)
        hipLaunchKernelGGL(k_quant_rows<1>, grid, dim3(64), 0, s, src, src_stride, n, dst, dst_stride, scale, rows);
    else if (chunks <= 512)
        hipLaunchKernelGGL(k_quant_rows<8>, grid, dim3(64), 0, s, src, src_stride, n, dst, dst_stride, scale, rows);
    else if (chunks <= 1024)
        hipLaunchKernelGGL(k_quant_rows<16>, grid, dim3(64), 0, s, src, src_stride, n, dst, dst_stride, scale, rows);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_pack_w13_e4m3(const void* const* w1, const void* const* w3, uint8_t* dst, int experts, int ffn,
                                int hidden, hipStream_t s) {
    const int KT = hidden / 128;
    const int64_t per_expert = static_cast<int64_t>(ffn / 64) * KT * 128 * 128;
    const dim3 grid(static_cast<unsigned>(ceil_div(per_expert, 256)));
    for (int e = 0; e < experts; ++e)
        hipLaunchKernelGGL(k_pack_tiles_e4m3, grid, dim3(256), 0, s, static_cast<const uint8_t*>(w1[e]),
                           static_cast<const uint8_t*>(w3[e]), dst + e * per_expert, hidden, KT, ffn / 64, 64);
    return hipGetLastError();
}

hipError_t launch_pack_w2_e4m3(const void* const* w2, uint8_t* dst, int experts, int ffn, int hidden,
                               hipStream_t s) {
    const int KT = static_cast<int>(ceil_div(ffn, 128));
    const int64_t per_expert = static_cast<int64_t>(hidden / 128) * KT * 128 * 128;
    const dim3 grid(static_cast<unsigned>(ceil_div(per_expert, 256)));
    for (int e = 0; e < experts; ++e)
        hipLaunchKernelGGL(k_pack_tiles_e4m3, grid, dim3(256), 0, s, static_cast<const uint8_t*>(w2[e]),
                           static_cast<const uint8_t*>(w2[e]), dst + e * per_expert, ffn, KT, hidden / 128, 128);
    return hipGetLastError();
}

}  // namespace aps
