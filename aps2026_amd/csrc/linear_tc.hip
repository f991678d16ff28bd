// Split-bf16 Linear on the bf16 matrix cores: the reference's optional
// tensor-core projection path.
//
// Reference: Tensor::prepare_cuda_bf16_weight and k_pack_bf16_weight
// (src/tensor.cu:124-177: W = W_hi + W_lo, W_hi = bf16(w), W_lo = bf16(w -
// W_hi), round to nearest even), k_matmul_transposed_bf16_wmma
// (src/tensor.cu:514-584: x split the same way on the fly; per 16-k step
// acc += x_hi W_hi + x_hi W_lo + x_lo W_hi, and x_lo W_lo as well under
// USE_TC_ALL; fp32 accumulation), its dispatch in matmul_transposed_gpu
// (src/tensor.cu:3042-3055) and the bias added after the product
// (matmul_transposed_bias_gpu, src/tensor.cu:3121-3142).  The sum is an
// approximation of the fp32 product (the dropped lo x lo term and the
// residual of lo are about 2^-16 of a product), accumulated in a different
// order than the fp32 chain, so it is compared with the fp32 oracle under a
// tolerance, not bit for bit.
//
// gfx950 mapping.
//  * x is split once into bf16 x_hi and x_lo row-major arrays (k_split_bf16,
//    shared by every projection of one input), W once at preparation into
//    the swizzled 128-row x 64-k tile images the MoE GEMMs use (hi images,
//    then lo images).
//  * A block computes 128 rows x 128 columns with four waves of 64 x 64
//    (v_mfma_f32_32x32x16_bf16, 2 x 2 tiles per wave).  A 64-k stage holds
//    x_hi, x_lo, W_hi and W_lo tiles: 512 rows of 128 bytes (64 KB), copied
//    with global_load_lds_dwordx4 into a two-stage LDS ring; the copy of stage
//    k + 1 runs while stage k is multiplied.  Per 16-k step a wave reads 8
//    operand fragments for 12 (16 with all terms) MFMAs.
//  * Rows past M and columns past N read clamped rows / zero-padded images
//    and are not stored.
#include "common.hpp"

namespace aps {
namespace {

typedef __bf16 tbf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 tbf16x2_t __attribute__((ext_vector_type(2)));
typedef float tf32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t tu32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTcRows = 128;                 // x rows per block
constexpr int kTcCols = 128;                 // output columns per block (one weight image)
constexpr int kTcRowBytes = 128;             // a stage row: 64 bf16
constexpr int kTcImage = 128 * kTcRowBytes;  // one packed weight image (16 KB)
constexpr int kTcStageRows = 4 * 128;        // x_hi, x_lo, W_hi, W_lo
constexpr int kTcStageBytes = kTcStageRows * kTcRowBytes;   // 64 KB

#define APS_TGP(p) ((const __attribute__((address_space(1))) void*)(p))
#define APS_TLP(p) ((__attribute__((address_space(3))) void*)(p))

// Byte offset of logical 16-byte chunk `chunk` of stage row `row`: the MoE
// GEMMs' swizzle (rows 2m, 2m + 1 share a 256-byte bank row; eight row
// pairs get eight different physical chunks).
__device__ inline int tswz(int row, int chunk) { return row * kTcRowBytes + ((chunk ^ ((row >> 1) & 7)) << 4); }

__device__ inline uint16_t bf16_bits(float v) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v)); }
__device__ inline float bf16_value(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// hi = bf16(v), lo = bf16(v - hi): v - hi is exact in fp32.
__device__ inline void split2(float v, uint16_t& hi, uint16_t& lo) {
    hi = bf16_bits(v);
    lo = bf16_bits(v - bf16_value(hi));
}

// x [n] fp32 -> hi, lo bf16; 8 elements per thread (n % 8 == 0).
__global__ void __launch_bounds__(256)
k_split_bf16(const float* __restrict__ x, uint16_t* __restrict__ hi, uint16_t* __restrict__ lo, int64_t n8) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n8) return;
    const float4 a = reinterpret_cast<const float4*>(x)[2 * i];
    const float4 b = reinterpret_cast<const float4*>(x)[2 * i + 1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint16_t h[8], l[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) split2(v[j], h[j], l[j]);
    tu32x4_t ph, pl;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        ph[j] = static_cast<uint32_t>(h[2 * j]) | (static_cast<uint32_t>(h[2 * j + 1]) << 16);
        pl[j] = static_cast<uint32_t>(l[2 * j]) | (static_cast<uint32_t>(l[2 * j + 1]) << 16);
    }
    reinterpret_cast<tu32x4_t*>(hi)[i] = ph;
    reinterpret_cast<tu32x4_t*>(lo)[i] = pl;
}

// W [N][K] fp32 -> images: image (nb * KT + kt) holds rows 128 nb .. + 127,
// k 64 kt .. + 63, swizzled; rows past N are zero.  hi images first, then
// lo images.  One thread per element.
__global__ void __launch_bounds__(256)
k_pack_split(const float* __restrict__ w, uint16_t* __restrict__ img, int N, int K, int64_t per_set) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= per_set) return;
    const int KT = K / 64;
    const int pk = static_cast<int>(i & 63);          // element in the physical row
    const int r = static_cast<int>((i >> 6) & 127);   // image row
    const int64_t t = i >> 13;                        // image index nb * KT + kt
    const int kt = static_cast<int>(t % KT);
    const int nb = static_cast<int>(t / KT);
    const int c = (pk >> 3) ^ ((r >> 1) & 7);         // logical chunk at this physical chunk
    const int k = kt * 64 + c * 8 + (pk & 7);
    const int64_t n = static_cast<int64_t>(nb) * 128 + r;
    const float v = n < N ? w[n * K + k] : 0.0f;
    uint16_t h, l;
    split2(v, h, l);
    img[i] = h;
    img[per_set + i] = l;
}

// Up to three outputs of one input (q, k and v): segment j is y[j]
// [M][n[j]] from packed weights w[j], column blocks t0[j] .. t0[j + 1] - 1 of
// the grid's x dimension.
struct TcSegs {
    const uint16_t* w[3];
    const float* b[3];
    float* y[3];
    int64_t per_set[3];
    int n[3];
    int t0[4];
};

// One-dimensional grid over the row-tile-major tile order, dealt to XCDs as
// k_linear_mfma's (workgroup b on XCD b % 8): tile b, or with xcd_rows tile
// (b % 8) * per + b / 8, so that the column tiles of a row tile share its x
// rows in one L2 (picked when x is the larger operand by 3x or more).
constexpr int kTcXcds = 8;

template <bool ALL>
__global__ void __launch_bounds__(256, 1)
k_linear_tc(const uint16_t* __restrict__ xhi, const uint16_t* __restrict__ xlo, const TcSegs segs, int64_t M,
            int K, int row_tiles, int xcd_rows) {
    __shared__ __align__(16) uint8_t ring[2][kTcStageBytes];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ncol = segs.t0[3];
    const int64_t per = (static_cast<int64_t>(row_tiles) * ncol + kTcXcds - 1) / kTcXcds;
    const int64_t t = xcd_rows ? static_cast<int64_t>(blockIdx.x % kTcXcds) * per + blockIdx.x / kTcXcds
                               : static_cast<int64_t>(blockIdx.x);
    if (t >= static_cast<int64_t>(row_tiles) * ncol) return;
    const int64_t m0 = (t / ncol) * kTcRows;
    // this block's segment (selects, so the argument block stays in scalar registers)
    const int bx = static_cast<int>(t % ncol);
    const int sg = (bx >= segs.t0[1]) + (bx >= segs.t0[2]);
    const uint16_t* __restrict__ img = sg == 0 ? segs.w[0] : sg == 1 ? segs.w[1] : segs.w[2];
    const float* __restrict__ bias = sg == 0 ? segs.b[0] : sg == 1 ? segs.b[1] : segs.b[2];
    float* __restrict__ y = sg == 0 ? segs.y[0] : sg == 1 ? segs.y[1] : segs.y[2];
    const int64_t per_set = sg == 0 ? segs.per_set[0] : sg == 1 ? segs.per_set[1] : segs.per_set[2];
    const int N = sg == 0 ? segs.n[0] : sg == 1 ? segs.n[1] : segs.n[2];
    const int nb = bx - (sg == 0 ? segs.t0[0] : sg == 1 ? segs.t0[1] : segs.t0[2]);
    const int KT = K / 64;
    const int64_t row_bytes = static_cast<int64_t>(K) * 2;

    // copy slots: instruction s (0..15) of wave w fills stage rows 32 s + 8 w
    // .. +7; lane i lands at physical chunk i & 7 of row 32 s + 8 w + i / 8.
    // Rows 0..127: x_hi, 128..255: x_lo (row-major, gathered per chunk),
    // 256..383: W_hi image rows, 384..511: W_lo image rows (pre-swizzled,
    // copied verbatim).
    const uint8_t* src[16];
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        const int row = 32 * s + 8 * wave + (lane >> 3);
        if (row < 256) {
            const int r = row & 127;
            const int64_t xr = m0 + r < M ? m0 + r : M - 1;
            const int chunk = (lane & 7) ^ ((row >> 1) & 7);
            const uint16_t* base = row < 128 ? xhi : xlo;
            src[s] = reinterpret_cast<const uint8_t*>(base) + xr * row_bytes + chunk * 16;
        } else {
            const int ir = (row - 256) & 127;
            const uint16_t* set = row < 384 ? img : img + per_set;
            src[s] = reinterpret_cast<const uint8_t*>(set) + static_cast<int64_t>(nb) * KT * kTcImage +
                     ir * kTcRowBytes + (lane & 7) * 16;
        }
    }
    auto issue = [&](uint8_t* st, int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const int64_t adv = s < 8 ? static_cast<int64_t>(kt) * kTcRowBytes : static_cast<int64_t>(kt) * kTcImage;
            __builtin_amdgcn_global_load_lds(APS_TGP(src[s] + adv), APS_TLP(st + (32 * s + 8 * wave) * kTcRowBytes),
                                             16, 0, 0);
        }
    };

    const int aR = (wave & 1) * 64, bR = (wave >> 1) * 64;
    tf32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = tf32x16_t{};

    auto frag = [&](const uint8_t* st, int row, int kk) __attribute__((always_inline)) {
        return __builtin_bit_cast(tbf16x8_t,
                                  *reinterpret_cast<const tu32x4_t*>(st + tswz(row, 2 * kk + (lane >> 5))));
    };
    issue(ring[0], 0);
    for (int kt = 0; kt < KT; ++kt) {
        uint8_t* st = ring[kt & 1];
        __builtin_amdgcn_s_waitcnt((0 & 0xF) | (0x7 << 4) | (0xF << 8));   // vmcnt(0): stage kt landed
        __syncthreads();                                                    // and every wave is past stage kt - 1
        if (kt + 1 < KT) issue(ring[(kt + 1) & 1], kt + 1);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            tbf16x8_t ah[2], al[2], bh[2], bl[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                ah[i] = frag(st, aR + 32 * i + (lane & 31), kk);
                al[i] = frag(st, 128 + aR + 32 * i + (lane & 31), kk);
                bh[i] = frag(st, 256 + bR + 32 * i + (lane & 31), kk);
                bl[i] = frag(st, 384 + bR + 32 * i + (lane & 31), kk);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bh[j], ah[i], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bl[j], ah[i], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bh[j], al[i], acc[i][j], 0, 0, 0);
                    if (ALL) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bl[j], al[i], acc[i][j], 0, 0, 0);
                }
        }
    }

    // W first in the MFMA: lane % 32 is an x row, register group q = v / 4
    // holds output columns 8 q + 4 (lane / 32) .. +3 of the 32-column tile
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int64_t row = m0 + aR + 32 * i + (lane & 31);
        if (row >= M) continue;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int col = nb * kTcCols + bR + 32 * j + 8 * q + 4 * (lane >> 5);
                if (col >= N) continue;   // N % 4 == 0: a group is all in or all out
                float4 o = make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                       acc[i][j][4 * q + 3]);
                if (bias) {
                    const float4 b = *reinterpret_cast<const float4*>(bias + col);
                    o = make_float4(__fadd_rn(o.x, b.x), __fadd_rn(o.y, b.y), __fadd_rn(o.z, b.z), __fadd_rn(o.w, b.w));
                }
                *reinterpret_cast<float4*>(y + row * N + col) = o;
            }
    }
}

}  // namespace

int64_t linear_tc_packed_elems(int out_f, int in_f) {
    // hi and lo image sets, each ceil(out / 128) * (in / 64) images of 128 x 64
    return 2 * ceil_div(out_f, 128) * (in_f / 64) * 128 * 64;
}

hipError_t launch_linear_tc_prepare(const float* w, int out_f, int in_f, uint16_t* packed, hipStream_t s) {
    if (out_f <= 0 || in_f <= 0 || in_f % 64 != 0) return hipErrorInvalidValue;
    const int64_t per_set = linear_tc_packed_elems(out_f, in_f) / 2;
    hipLaunchKernelGGL(k_pack_split, dim3(static_cast<unsigned>(ceil_div(per_set, 256))), dim3(256), 0, s, w, packed,
                       out_f, in_f, per_set);
    return hipGetLastError();
}

hipError_t launch_split_bf16(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (n % 8 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_split_bf16, dim3(static_cast<unsigned>(ceil_div(n / 8, 256))), dim3(256), 0, s, x, hi, lo,
                       n / 8);
    return hipGetLastError();
}

hipError_t launch_linear_tc_multi(const uint16_t* xhi, const uint16_t* xlo, int count, const uint16_t* const* packed,
                                  const float* const* bias, float* const* y, const int* out_f, int64_t rows, int in_f,
                                  bool all_terms, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (count < 1 || count > 3 || in_f <= 0 || in_f % 64 != 0 || ceil_div(rows, kTcRows) > 65535)
        return hipErrorInvalidValue;
    TcSegs segs{};
    int t = 0;
    for (int j = 0; j < 3; ++j) {
        segs.t0[j] = t;
        const int jj = j < count ? j : 0;   // unused segments: never selected (their t0 is the tile count)
        if (out_f[jj] <= 0 || out_f[jj] % 4 != 0) return hipErrorInvalidValue;
        segs.w[j] = packed[jj];
        segs.b[j] = bias[jj];
        segs.y[j] = y[jj];
        segs.n[j] = out_f[jj];
        segs.per_set[j] = linear_tc_packed_elems(out_f[jj], in_f) / 2;
        if (j < count) t += static_cast<int>(ceil_div(out_f[j], kTcCols));
    }
    segs.t0[3] = t;
    for (int j = count; j < 3; ++j) segs.t0[j] = t;
    const int64_t rt = ceil_div(rows, kTcRows);
    int64_t wcols = 0;
    for (int j = 0; j < count; ++j) wcols += out_f[j];
    const int xr = rows >= 3 * wcols ? 1 : 0;   // x bytes >= 3 x W bytes (both hi + lo bf16)
    const dim3 grid(static_cast<unsigned>(ceil_div(rt * t, kTcXcds) * kTcXcds));
    if (all_terms)
        hipLaunchKernelGGL(k_linear_tc<true>, grid, dim3(256), 0, s, xhi, xlo, segs, rows, in_f, static_cast<int>(rt), xr);
    else
        hipLaunchKernelGGL(k_linear_tc<false>, grid, dim3(256), 0, s, xhi, xlo, segs, rows, in_f, static_cast<int>(rt), xr);
    return hipGetLastError();
}

hipError_t launch_linear_tc(const uint16_t* xhi, const uint16_t* xlo, const uint16_t* packed, const float* bias,
                            float* y, int64_t rows, int in_f, int out_f, bool all_terms, hipStream_t s) {
    return launch_linear_tc_multi(xhi, xlo, 1, &packed, &bias, &y, &out_f, rows, in_f, all_terms, s);
}

}  // namespace aps
