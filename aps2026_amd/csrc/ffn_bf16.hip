// Grouped expert FFN on gfx950 bf16 MFMA (fp32 accumulate).
//
// Reference: k_moe_pair_silu_8x8 (src/tensor.cu:1838-1966) computes
// silu(x . w1^T) * (x . w3^T) for each expert's row range with the gather
// folded into the A load (assignment_rows), and k_moe_matmul_8x8
// (src/tensor.cu:1740-1836) multiplies by w2^T.  Both are fp32 SIMT GEMMs
// over a 128-row work list (src/tensor.cu:1333-1374).
//
// gfx950 design.
//  * MFMA v_mfma_f32_32x32x16_bf16: each wave owns a 64-row x 64-col output
//    tile (2x2 MFMA tiles, 64 fp32 accumulators per lane); four waves form a
//    128 x 128 output tile.  In the w1||w3 kernel the 128 columns are 64
//    gate and the SAME 64 up columns, so SiLU(g)*u closes inside each lane.
//  * A and B tiles (128 rows x 64 k, bf16) go through LDS, double buffered
//    with register prefetch; 16-byte chunks are XOR-swizzled by (row & 7) so
//    that both the row-contiguous global->LDS stores and the per-lane
//    ds_read_b128 MFMA operand fetches are bank-conflict free.
//  * w1 and w3 are re-packed at registration to [E][F/64][128][H]: the 64
//    gate rows and 64 up rows of one column block are one contiguous 1 MB
//    slab, so the B tile of a block is a single strided stream.
//  * The token gather of the w1||w3 kernel is an index on the A load, as in
//    the reference: no permuted copy of x is ever written.
//  * Work list: blockIdx.y is a linear row-tile index over all experts
//    (sum_e ceil(count_e / 128) tiles); each block finds its expert from
//    offsets[] with a wave-uniform scan (scalar loads), so skewed experts
//    simply own more tiles and no host round trip is needed.
#include "common.hpp"

namespace aps {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
// native vector (not HIP's uint4 struct, whose copies become memcpy through
// a stack slot): 16 bytes = one ds_read_b128 / global_load_dwordx4
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;        // k per LDS stage
constexpr int kTileRows = 128; // rows of an LDS operand tile

// Element offset of 16-byte chunk `chunk` (0..7) of tile row `row`.
__device__ inline int swz(int row, int chunk) { return row * kBK + ((chunk ^ (row & 7)) << 3); }

__device__ inline bf16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<bf16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<bf16_t>(u >> 16);
}

__device__ inline bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ inline f32x16_t mfma(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Finds (expert, first position, end position) of row tile `tile` of size
// `bm`; returns false when the tile index is past the last tile.
__device__ inline bool locate_tile(const uint32_t* __restrict__ offsets, int E, int tile, int bm,
                                   int& expert, uint32_t& m0, uint32_t& end) {
    int cum = 0;
    for (int e = 0; e < E; ++e) {
        const uint32_t lo = offsets[e], hi = offsets[e + 1];
        const int nt = static_cast<int>((hi - lo + bm - 1) / bm);
        if (tile < cum + nt) {
            expert = e;
            m0 = lo + static_cast<uint32_t>(tile - cum) * bm;
            end = hi;
            return true;
        }
        cum += nt;
    }
    return false;
}

// The 32x32 MFMA accumulator layout: register v of lane l holds
// D[row(v, l)][l % 32] with row = 8 * (v / 4) + 4 * (l / 32) + v % 4.
__device__ inline int acc_row(int v, int lane) { return ((v >> 2) << 3) + ((lane >> 5) << 2) + (v & 3); }

// silu(g) * u for the bf16 path (fp32 math, hardware exp2).
__device__ inline float swiglu(float g, float u) {
    return g / (1.0f + __expf(-g)) * u;
}

// ---------------------------------------------------------------------------
// act[p][n] = silu(x[t] . w1[e][n]) * (x[t] . w3[e][n]),  t = assignment_rows[p]
__global__ void __launch_bounds__(256, 2)
k_ffn_up_bf16(const bf16_t* __restrict__ x, const uint32_t* __restrict__ offsets,
              const uint32_t* __restrict__ assignment_rows, const bf16_t* __restrict__ w13,
              bf16_t* __restrict__ act, int H, int F, int E) {
    __shared__ __align__(16) bf16_t As[2][kTileRows * kBK];
    __shared__ __align__(16) bf16_t Bs[2][kTileRows * kBK];

    int e;
    uint32_t m0, end;
    if (!locate_tile(offsets, E, blockIdx.y, kUpBM, e, m0, end)) return;
    const int nb = blockIdx.x;  // 64-column block of the intermediate dim

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lc = tid & 7, lr = tid >> 3;

    // Per-thread load addressing as vector values (kept in registers): the
    // four A rows this thread stages are tokens a_tok[j] (or -1 past the
    // expert's last row); B rows are lr + 32j of the block's 128-row slab.
    i32x4_t a_tok;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t p = m0 + lr + 32 * j;
        a_tok[j] = p < end ? static_cast<int>(assignment_rows[p]) : -1;
    }
    const bf16_t* b_ptr = w13 + (static_cast<int64_t>(e) * (F / kUpBN) + nb) * 128 * static_cast<int64_t>(H) +
                          static_cast<int64_t>(lr) * H + lc * 8;
    const int64_t b_step = 32 * static_cast<int64_t>(H);
    u32x4_t ra[4], rb[4];
    auto gload = [&](int k0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int tok = a_tok[j];
            ra[j] = tok >= 0 ? *reinterpret_cast<const u32x4_t*>(x + static_cast<int64_t>(tok) * H + k0 + lc * 8)
                             : u32x4_t{0u, 0u, 0u, 0u};
            rb[j] = *reinterpret_cast<const u32x4_t*>(b_ptr + j * b_step + k0);
        }
    };
    auto lstore = [&](int st) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = lr + 32 * j;
            *reinterpret_cast<u32x4_t*>(&As[st][swz(row, lc)]) = ra[j];
            *reinterpret_cast<u32x4_t*>(&Bs[st][swz(row, lc)]) = rb[j];
        }
    };

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][h][v] = 0.0f;

    const int KT = H / kBK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int st = kt & 1;
        if (kt + 1 < KT) gload((kt + 1) * kBK);
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            const int chunk = kk * 2 + (lane >> 5);
            bf16x8_t af[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = wm * 64 + i * 32 + (lane & 31);
                af[i] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&As[st][swz(row, chunk)]));
            }
            const int bg_row = wn * 32 + (lane & 31);
            const bf16x8_t bg = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&Bs[st][swz(bg_row, chunk)]));
            const bf16x8_t bu = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&Bs[st][swz(bg_row + 64, chunk)]));
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                acc[i][0] = mfma(af[i], bg, acc[i][0]);
                acc[i][1] = mfma(af[i], bu, acc[i][1]);
            }
        }
        if (kt + 1 < KT) lstore(st ^ 1);
        __syncthreads();
    }

    const int col = nb * kUpBN + wn * 32 + (lane & 31);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint32_t p = m0 + wm * 64 + i * 32 + acc_row(v, lane);
            if (p < end) act[static_cast<int64_t>(p) * F + col] = f32_to_bf16(swiglu(acc[i][0][v], acc[i][1][v]));
        }
    }
}

// ---------------------------------------------------------------------------
// y[p][n] = act[p] . w2[e][n]
__global__ void __launch_bounds__(256, 2)
k_ffn_down_bf16(const bf16_t* __restrict__ act, const uint32_t* __restrict__ offsets,
                const bf16_t* __restrict__ w2, bf16_t* __restrict__ y, int H, int F, int E) {
    __shared__ __align__(16) bf16_t As[2][kTileRows * kBK];
    __shared__ __align__(16) bf16_t Bs[2][kTileRows * kBK];

    int e;
    uint32_t m0, end;
    if (!locate_tile(offsets, E, blockIdx.y, kDownBM, e, m0, end)) return;
    const int nb = blockIdx.x;  // 128-column block of the hidden dim

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lc = tid & 7, lr = tid >> 3;

    // A rows m0 + lr + 32j are live while below `end`; B rows are hidden
    // columns nb*128 + lr + 32j of w2[e].
    const uint32_t a_row0 = m0 + lr;
    const bf16_t* a_ptr = act + static_cast<int64_t>(a_row0) * F + lc * 8;
    const int64_t a_step = 32 * static_cast<int64_t>(F);
    const bf16_t* b_ptr = w2 + (static_cast<int64_t>(e) * H + static_cast<int64_t>(nb) * kDownBN + lr) * F + lc * 8;
    const int64_t b_step = 32 * static_cast<int64_t>(F);
    u32x4_t ra[4], rb[4];
    auto gload = [&](int k0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            ra[j] = a_row0 + 32 * j < end ? *reinterpret_cast<const u32x4_t*>(a_ptr + j * a_step + k0)
                                          : u32x4_t{0u, 0u, 0u, 0u};
            rb[j] = *reinterpret_cast<const u32x4_t*>(b_ptr + j * b_step + k0);
        }
    };
    auto lstore = [&](int st) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = lr + 32 * j;
            *reinterpret_cast<u32x4_t*>(&As[st][swz(row, lc)]) = ra[j];
            *reinterpret_cast<u32x4_t*>(&Bs[st][swz(row, lc)]) = rb[j];
        }
    };

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][h][v] = 0.0f;

    const int KT = F / kBK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int st = kt & 1;
        if (kt + 1 < KT) gload((kt + 1) * kBK);
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            const int chunk = kk * 2 + (lane >> 5);
            bf16x8_t af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = wm * 64 + i * 32 + (lane & 31);
                af[i] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&As[st][swz(row, chunk)]));
                const int brow = wn * 64 + i * 32 + (lane & 31);
                bf[i] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&Bs[st][swz(brow, chunk)]));
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma(af[i], bf[j], acc[i][j]);
        }
        if (kt + 1 < KT) lstore(st ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t col = static_cast<int64_t>(nb) * kDownBN + wn * 64 + j * 32 + (lane & 31);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t p = m0 + wm * 64 + i * 32 + acc_row(v, lane);
                if (p < end) y[static_cast<int64_t>(p) * H + col] = f32_to_bf16(acc[i][j][v]);
            }
        }
    }
}

}  // namespace

hipError_t launch_ffn_up_bf16(const bf16_t* x, const uint32_t* offsets,
                              const uint32_t* assignment_rows, const bf16_t* w13,
                              bf16_t* act, int64_t rows, int hidden, int ffn, int experts,
                              hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hidden % kBK != 0 || ffn % kUpBN != 0) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(ffn / kUpBN),
                    static_cast<unsigned>(max_row_tiles(2 * rows, kUpBM, experts)));
    hipLaunchKernelGGL(k_ffn_up_bf16, grid, dim3(256), 0, s, x, offsets, assignment_rows, w13, act,
                       hidden, ffn, experts);
    return hipGetLastError();
}

hipError_t launch_ffn_down_bf16(const bf16_t* act, const uint32_t* offsets, const bf16_t* w2,
                                bf16_t* y, int64_t rows, int hidden, int ffn, int experts,
                                hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hidden % kDownBN != 0 || ffn % kBK != 0) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(hidden / kDownBN),
                    static_cast<unsigned>(max_row_tiles(2 * rows, kDownBM, experts)));
    hipLaunchKernelGGL(k_ffn_down_bf16, grid, dim3(256), 0, s, act, offsets, w2, y, hidden, ffn,
                       experts);
    return hipGetLastError();
}

}  // namespace aps
