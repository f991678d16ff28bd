// Grouped expert FFN in fp32 with the reference's accumulation order.
//
// Reference: k_moe_pair_silu_8x8 (src/tensor.cu:1838-1966) and
// k_moe_matmul_8x8 (src/tensor.cu:1740-1836) give every output ONE fp32
// accumulator walked over k ascending with FMA (nvcc contracts
// `acc += a * b`), and the SiLU epilogue evaluates exp in double:
// a = g / (1 + (float)exp((double)-g)) * u.
//
// These kernels keep exactly that arithmetic, so for fp32 weights the result
// equals the CPU oracle bit for bit (the only libm call, exp in double, is
// rounded to float afterwards).  They are SIMT kernels: each thread owns a
// 4 x 4 block of outputs per operand and walks k in order; operand tiles are
// staged k-major in LDS so the inner step is three ds_read_b128 + 32 FMAs.
// This is the exactness path (config C1, fp32); the throughput path is
// the bf16 MFMA kernel.
#include "common.hpp"

namespace aps {
namespace {

constexpr int kBK = 16;

__device__ inline bool locate_tile(const uint32_t* __restrict__ offsets, int E, int tile, int bm,
                                   int& expert, uint32_t& m0, uint32_t& end) {
    uint32_t lo, hi;
    int incl;
    const int total = wave_tile_scan(offsets, E, bm, lo, hi, incl);
    if (tile >= total) return false;
    const RowTile r = wave_find_tile(tile, bm, lo, hi, incl, E);
    expert = r.expert;
    m0 = r.m0;
    end = r.end;
    return true;
}

// a = g / (1 + (float)exp((double)-g)) * u, each operation rounded on its own
// (src/tensor.cu:1961-1963, src/layer.cu:8-11).
__device__ inline float swiglu_exact(float g, float u) {
    const float ex = static_cast<float>(exp(-static_cast<double>(g)));
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, ex)), u);
}

// 64 rows x 64 intermediate columns of gate AND up per block.
__global__ void __launch_bounds__(256)
k_ffn_up_f32(const float* __restrict__ x, const uint32_t* __restrict__ offsets,
             const uint32_t* __restrict__ assignment_rows, const float* __restrict__ w1,
             const float* __restrict__ w3, float* __restrict__ act, int H, int F, int E) {
    __shared__ __align__(16) float As[kBK][kF32BM];
    __shared__ __align__(16) float Gs[kBK][kF32BN];
    __shared__ __align__(16) float Us[kBK][kF32BN];

    int e;
    uint32_t m0, end;
    if (!locate_tile(offsets, E, blockIdx.y, kF32BM, e, m0, end)) return;
    const int n0 = blockIdx.x * kF32BN;
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    // staging: one float4 of A, of w1 and of w3 per thread per k tile
    const int sr = tid >> 2, sk = (tid & 3) * 4;
    const uint32_t p = m0 + sr;
    const bool a_ok = p < end;
    const float* a_src = x + static_cast<int64_t>(a_ok ? assignment_rows[p] : 0) * H + sk;
    const bool b_ok = n0 + sr < F;
    const int64_t brow = static_cast<int64_t>(e) * F + (b_ok ? n0 + sr : 0);
    const float* g_src = w1 + brow * H + sk;
    const float* u_src = w3 + brow * H + sk;

    float ga[4][4], ua[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) { ga[r][c] = 0.0f; ua[r][c] = 0.0f; }

    for (int k0 = 0; k0 < H; k0 += kBK) {
        const float4 av = a_ok ? *reinterpret_cast<const float4*>(a_src + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 gv = b_ok ? *reinterpret_cast<const float4*>(g_src + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 uv = b_ok ? *reinterpret_cast<const float4*>(u_src + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
        __syncthreads();
        As[sk + 0][sr] = av.x; As[sk + 1][sr] = av.y; As[sk + 2][sr] = av.z; As[sk + 3][sr] = av.w;
        Gs[sk + 0][sr] = gv.x; Gs[sk + 1][sr] = gv.y; Gs[sk + 2][sr] = gv.z; Gs[sk + 3][sr] = gv.w;
        Us[sk + 0][sr] = uv.x; Us[sk + 1][sr] = uv.y; Us[sk + 2][sr] = uv.z; Us[sk + 3][sr] = uv.w;
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kBK; ++kk) {
            const float4 a = *reinterpret_cast<const float4*>(&As[kk][ty * 4]);
            const float4 g = *reinterpret_cast<const float4*>(&Gs[kk][tx * 4]);
            const float4 u = *reinterpret_cast<const float4*>(&Us[kk][tx * 4]);
            const float ar[4] = {a.x, a.y, a.z, a.w};
            const float gr[4] = {g.x, g.y, g.z, g.w};
            const float ur[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    ga[r][c] = __builtin_fmaf(ar[r], gr[c], ga[r][c]);
                    ua[r][c] = __builtin_fmaf(ar[r], ur[c], ua[r][c]);
                }
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t pr = m0 + ty * 4 + r;
        if (pr >= end) continue;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int col = n0 + tx * 4 + c;
            if (col < F) act[static_cast<int64_t>(pr) * F + col] = swiglu_exact(ga[r][c], ua[r][c]);
        }
    }
}

// 64 rows x 64 hidden columns per block; K = F walked ascending.
__global__ void __launch_bounds__(256)
k_ffn_down_f32(const float* __restrict__ act, const uint32_t* __restrict__ offsets,
               const float* __restrict__ w2, float* __restrict__ y, int H, int F, int E) {
    __shared__ __align__(16) float As[kBK][kF32BM];
    __shared__ __align__(16) float Bs[kBK][kF32BN];

    int e;
    uint32_t m0, end;
    if (!locate_tile(offsets, E, blockIdx.y, kF32BM, e, m0, end)) return;
    const int n0 = blockIdx.x * kF32BN;
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int sr = tid >> 2, sk = (tid & 3) * 4;
    const uint32_t p = m0 + sr;
    const bool a_ok = p < end;
    const float* a_src = act + static_cast<int64_t>(a_ok ? p : m0) * F + sk;
    const bool b_ok = n0 + sr < H;
    const float* b_src = w2 + (static_cast<int64_t>(e) * H + (b_ok ? n0 + sr : 0)) * F + sk;

    float acc[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[r][c] = 0.0f;

    for (int k0 = 0; k0 < F; k0 += kBK) {
        const float4 av = a_ok ? *reinterpret_cast<const float4*>(a_src + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 bv = b_ok ? *reinterpret_cast<const float4*>(b_src + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
        __syncthreads();
        As[sk + 0][sr] = av.x; As[sk + 1][sr] = av.y; As[sk + 2][sr] = av.z; As[sk + 3][sr] = av.w;
        Bs[sk + 0][sr] = bv.x; Bs[sk + 1][sr] = bv.y; Bs[sk + 2][sr] = bv.z; Bs[sk + 3][sr] = bv.w;
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kBK; ++kk) {
            const float4 a = *reinterpret_cast<const float4*>(&As[kk][ty * 4]);
            const float4 b = *reinterpret_cast<const float4*>(&Bs[kk][tx * 4]);
            const float ar[4] = {a.x, a.y, a.z, a.w};
            const float br[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[r][c] = __builtin_fmaf(ar[r], br[c], acc[r][c]);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t pr = m0 + ty * 4 + r;
        if (pr >= end) continue;
        const int col = n0 + tx * 4;
        if (col + 3 < H)
            *reinterpret_cast<float4*>(y + static_cast<int64_t>(pr) * H + col) =
                make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
    }
}

// y[m][n] = (fp32 FMA chain over k ascending of x[m][k] w[n][k]) + bias[n]:
// the decoder's Linear layers (the attention projections).  Reference:
// Linear::forward (src/layer.cu:30-42) -> matmul_transposed_bias_gpu
// (src/tensor.cu:3120-3143) -> k_matmul_transposed_8x8 (src/tensor.cu:
// 715-800): one accumulator per output walked over k ascending, the bias
// added once in the epilogue (nothing added without a bias).  64 x 64
// outputs per block, 4 x 4 per thread, as the expert kernels above.
__global__ void __launch_bounds__(256)
k_linear_f32(const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ bias,
             float* __restrict__ y, int64_t M, int K, int N) {
    __shared__ __align__(16) float As[kBK][kF32BM];
    __shared__ __align__(16) float Bs[kBK][kF32BN];
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kF32BM;
    const int n0 = blockIdx.x * kF32BN;
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int sr = tid >> 2, sk = (tid & 3) * 4;
    const bool a_ok = m0 + sr < M;
    const float* a_src = x + (a_ok ? m0 + sr : 0) * static_cast<int64_t>(K) + sk;
    const bool b_ok = n0 + sr < N;
    const float* b_src = w + static_cast<int64_t>(b_ok ? n0 + sr : 0) * K + sk;
    float acc[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[r][c] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += kBK) {
        const float4 av = a_ok ? *reinterpret_cast<const float4*>(a_src + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 bv = b_ok ? *reinterpret_cast<const float4*>(b_src + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
        __syncthreads();
        As[sk + 0][sr] = av.x; As[sk + 1][sr] = av.y; As[sk + 2][sr] = av.z; As[sk + 3][sr] = av.w;
        Bs[sk + 0][sr] = bv.x; Bs[sk + 1][sr] = bv.y; Bs[sk + 2][sr] = bv.z; Bs[sk + 3][sr] = bv.w;
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kBK; ++kk) {
            const float4 a = *reinterpret_cast<const float4*>(&As[kk][ty * 4]);
            const float4 b = *reinterpret_cast<const float4*>(&Bs[kk][tx * 4]);
            const float ar[4] = {a.x, a.y, a.z, a.w};
            const float br[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[r][c] = __builtin_fmaf(ar[r], br[c], acc[r][c]);
        }
    }
    const int col = n0 + tx * 4;  // N % 4 == 0: a column group is all in or all out
    float4 bb = make_float4(0.f, 0.f, 0.f, 0.f);
    if (bias && col < N) bb = *reinterpret_cast<const float4*>(bias + col);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t row = m0 + ty * 4 + r;
        if (row >= M || col >= N) continue;
        float4 o = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
        if (bias) o = make_float4(__fadd_rn(o.x, bb.x), __fadd_rn(o.y, bb.y), __fadd_rn(o.z, bb.z), __fadd_rn(o.w, bb.w));
        *reinterpret_cast<float4*>(y + row * N + col) = o;
    }
}

// The same product for any K, N and alignment (the reference's fallback for
// shapes its fast kernels do not take, k_matmul_transposed_tiled,
// src/tensor.cu:433-461): scalar loads, k past K read as zero.  A padded step
// adds the exact product 0 * 0 to an accumulator that is never -0 (it starts
// at +0, and a sum that cancels exactly rounds to +0), so it changes no bit:
// every output is the chain over k = 0 .. K-1.  Row tiles are walked
// grid-stride over gridDim.y.
__global__ void __launch_bounds__(256)
k_linear_any(const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ bias,
             float* __restrict__ y, int64_t M, int K, int N) {
    __shared__ float As[kBK][kF32BM + 1];
    __shared__ float Bs[kBK][kF32BN + 1];
    const int n0 = blockIdx.x * kF32BN;
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int sr = tid >> 2, sk = (tid & 3) * 4;
    const bool b_ok = n0 + sr < N;
    const float* b_src = w + static_cast<int64_t>(b_ok ? n0 + sr : 0) * K;
    for (int64_t m0 = static_cast<int64_t>(blockIdx.y) * kF32BM; m0 < M;
         m0 += static_cast<int64_t>(gridDim.y) * kF32BM) {
        const bool a_ok = m0 + sr < M;
        const float* a_src = x + (a_ok ? m0 + sr : 0) * static_cast<int64_t>(K);
        float acc[4][4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[r][c] = 0.0f;
        for (int k0 = 0; k0 < K; k0 += kBK) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int k = k0 + sk + i;
                av[i] = a_ok && k < K ? a_src[k] : 0.0f;
                bv[i] = b_ok && k < K ? b_src[k] : 0.0f;
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                As[sk + i][sr] = av[i];
                Bs[sk + i][sr] = bv[i];
            }
            __syncthreads();
#pragma unroll
            for (int kk = 0; kk < kBK; ++kk) {
                float ar[4], br[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    ar[i] = As[kk][ty * 4 + i];
                    br[i] = Bs[kk][tx * 4 + i];
                }
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[r][c] = __builtin_fmaf(ar[r], br[c], acc[r][c]);
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = m0 + ty * 4 + r;
            if (row >= M) continue;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int col = n0 + tx * 4 + c;
                if (col >= N) continue;
                y[row * N + col] = bias ? __fadd_rn(acc[r][c], bias[col]) : acc[r][c];
            }
        }
    }
}

}  // namespace

hipError_t launch_linear_f32(const float* x, const float* w, const float* bias, float* y, int64_t rows, int in_f,
                             int out_f, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    // the matrix-core kernel computes the same chains (see linear_mfma.hip);
    // this SIMT kernel serves in_f not a multiple of 32
    if (linear_mfma_fits(rows, in_f, out_f)) return launch_linear_mfma_f32(x, w, bias, y, rows, in_f, out_f, s);
    if (in_f % kBK != 0 || out_f % 4 != 0 || out_f <= 0) return hipErrorInvalidValue;
    const int64_t ty = ceil_div(rows, kF32BM);
    if (ty > 65535) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(ceil_div(out_f, kF32BN)), static_cast<unsigned>(ty));
    hipLaunchKernelGGL(k_linear_f32, grid, dim3(256), 0, s, x, w, bias, y, rows, in_f, out_f);
    return hipGetLastError();
}

hipError_t launch_linear_any_f32(const float* x, const float* w, const float* bias, float* y, int64_t rows, int in_f,
                                 int out_f, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (in_f <= 0 || out_f <= 0) return hipErrorInvalidValue;
    const int64_t ty = ceil_div(rows, kF32BM);
    const dim3 grid(static_cast<unsigned>(ceil_div(out_f, kF32BN)), static_cast<unsigned>(ty < 65535 ? ty : 65535));
    hipLaunchKernelGGL(k_linear_any, grid, dim3(256), 0, s, x, w, bias, y, rows, in_f, out_f);
    return hipGetLastError();
}

hipError_t launch_ffn_up_f32(const float* x, const uint32_t* offsets,
                             const uint32_t* assignment_rows, const float* w1,
                             const float* w3, float* act, int64_t rows, int hidden, int ffn,
                             int experts, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hidden % kBK != 0 || ffn % 4 != 0) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(ceil_div(ffn, kF32BN)),
                    static_cast<unsigned>(max_row_tiles(2 * rows, kF32BM, experts)));
    hipLaunchKernelGGL(k_ffn_up_f32, grid, dim3(256), 0, s, x, offsets, assignment_rows, w1, w3,
                       act, hidden, ffn, experts);
    return hipGetLastError();
}

hipError_t launch_ffn_down_f32(const float* act, const uint32_t* offsets, const float* w2,
                               float* y, int64_t rows, int hidden, int ffn, int experts,
                               hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (ffn % kBK != 0 || hidden % kF32BN != 0) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(hidden / kF32BN),
                    static_cast<unsigned>(max_row_tiles(2 * rows, kF32BM, experts)));
    hipLaunchKernelGGL(k_ffn_down_f32, grid, dim3(256), 0, s, act, offsets, w2, y, hidden, ffn,
                       experts);
    return hipGetLastError();
}

}  // namespace aps
