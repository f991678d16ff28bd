// Router: logits GEMM (bit-exact fp32 FMA chains) and quantised greedy top-2.
//
// Reference: k_matmul_transposed_narrow (src/tensor.cu:2943-3006) computes
// each logit as ONE fp32 accumulator walked over k = 0..H-1 with FMA, and
// k_moe_top2 (src/tensor.cu:1293-1331) quantises and greedy-selects.  The
// reference's own logs show that a last-ulp change upstream flips experts, so
// the chain order is fixed: no split-K, no tree reduction over k.
//
// gfx950 mapping.  The parallelism is T*E independent chains of length H.
// One lane owns one chain: a wavefront is 64 tokens x 1 expert.
//  * x: the 64 x 256 tile is staged once per workgroup in LDS as fp32 and
//    each lane reads its own row with ds_read_b128 (row pitch 260 floats:
//    the 16 lanes of an LDS phase land on 16 distinct 4-bank groups).
//  * gate: the value of step k is the same for the whole wave, so the
//    block's 4 x 256 gate chunk is staged in LDS beside x and every lane
//    reads it with the same address (an LDS broadcast).  Keeping both
//    operands in LDS puts all operand reads under the in-order LDS counter:
//    the reads of the next 16 steps are issued before the current 16 FMAs
//    (explicit ping-pong).  Scalar gate loads would return out of order and
//    force a full lgkmcnt wait at every prefetch.
//  * The chain is one dependent v_fmac_f32 per step; on gfx950 that issues
//    about every 9 cycles, which bounds this kernel at T = 4096 (one chain
//    per lane, one wave per SIMD).
// Four waves (four experts) share an x tile; the grid is [token tiles] x
// [E/4], and with tiles % 8 == 0 the four expert groups of a tile land on one
// XCD (blocks are dealt round-robin over the 8 XCDs), so x is fetched from
// HBM once per XCD L2.  The next 256-wide chunk of x and gate is
// prefetched into registers while the current one is consumed.
#include "common.hpp"

namespace aps {
namespace {

constexpr int kRouterKC = 256;              // k per LDS chunk
constexpr int kRouterPitch = kRouterKC + 4; // floats per LDS row
constexpr int kRouterExpertsPerBlock = 4;   // one wave per expert

// Loads one 64 x 256 chunk of x into registers, 4 consecutive k per piece:
// 4096 pieces, 16 per thread, piece p = row p / 64, columns 4 * (p % 64).
// Sixteen consecutive lanes therefore store 256 contiguous LDS bytes (one
// float4 each), which covers the 64 banks once: conflict-free.
template <bool XBF16>
struct XStage;

template <>
struct XStage<true> {
    static constexpr int kPieces = 16;
    uint2 v[kPieces];
    __device__ void load(const bf16_t* x, int64_t row0, int64_t rows, int H, int k0) {
#pragma unroll
        for (int j = 0; j < kPieces; ++j) {
            const int p = threadIdx.x + j * 256;
            const int64_t row = row0 + (p >> 6);
            v[j] = row < rows ? *reinterpret_cast<const uint2*>(x + row * H + k0 + (p & 63) * 4)
                              : make_uint2(0, 0);
        }
    }
    __device__ void store(float* xs) const {
#pragma unroll
        for (int j = 0; j < kPieces; ++j) {
            const int p = threadIdx.x + j * 256;
            *reinterpret_cast<float4*>(xs + (p >> 6) * kRouterPitch + (p & 63) * 4) =
                make_float4(__uint_as_float(v[j].x << 16), __uint_as_float(v[j].x & 0xffff0000u),
                            __uint_as_float(v[j].y << 16), __uint_as_float(v[j].y & 0xffff0000u));
        }
    }
};

template <>
struct XStage<false> {
    static constexpr int kPieces = 16;
    float4 v[kPieces];
    __device__ void load(const float* x, int64_t row0, int64_t rows, int H, int k0) {
#pragma unroll
        for (int j = 0; j < kPieces; ++j) {
            const int p = threadIdx.x + j * 256;
            const int64_t row = row0 + (p >> 6);
            v[j] = row < rows ? *reinterpret_cast<const float4*>(x + row * H + k0 + (p & 63) * 4)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    __device__ void store(float* xs) const {
#pragma unroll
        for (int j = 0; j < kPieces; ++j) {
            const int p = threadIdx.x + j * 256;
            *reinterpret_cast<float4*>(xs + (p >> 6) * kRouterPitch + (p & 63) * 4) = v[j];
        }
    }
};

// 16 chain steps acc = fma(x_k, g_k, acc), k ascending, one fused
// multiply-add each (v_fmac_f32); g comes from a wave-uniform LDS broadcast.
__device__ inline float fma16(float acc, const float4 (&x)[4], const float4 (&g)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        acc = __builtin_fmaf(x[i].x, g[i].x, acc);
        acc = __builtin_fmaf(x[i].y, g[i].y, acc);
        acc = __builtin_fmaf(x[i].z, g[i].z, acc);
        acc = __builtin_fmaf(x[i].w, g[i].w, acc);
    }
    return acc;
}

template <bool XBF16>
__global__ void __launch_bounds__(256, 2)
k_router_logits(const void* __restrict__ xv, const float* __restrict__ gate, int64_t rows,
                int H, int E, float* __restrict__ logits) {
    using XT = typename std::conditional<XBF16, bf16_t, float>::type;
    const XT* __restrict__ x = static_cast<const XT*>(xv);
    __shared__ __align__(16) float xs[kWave * kRouterPitch];
    __shared__ __align__(16) float gs[kRouterExpertsPerBlock][kRouterKC];

    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int e = blockIdx.y * kRouterExpertsPerBlock + w;
    const bool active = e < E;  // wave-uniform
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kWave;
    const float* xrow = xs + lane * kRouterPitch;
    const float* grow = gs[w];
    // gate staging: thread i copies float4 i of the block's 4 x 256 chunk
    const int ge = blockIdx.y * kRouterExpertsPerBlock + (threadIdx.x >> 6);
    const float* gsrc = gate + static_cast<int64_t>(ge < E ? ge : 0) * H + (threadIdx.x & 63) * 4;

    auto load_xg = [&](float4 (&xd)[4], float4 (&gd)[4], int kk) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xd[i] = *reinterpret_cast<const float4*>(xrow + kk + 4 * i);
            gd[i] = *reinterpret_cast<const float4*>(grow + kk + 4 * i);  // same address on every lane
        }
    };

    XStage<XBF16> st;
    float4 gv;
    st.load(x, row0, rows, H, 0);
    gv = *reinterpret_cast<const float4*>(gsrc);
    float acc = 0.0f;
    for (int k0 = 0; k0 < H; k0 += kRouterKC) {
        __syncthreads();  // previous chunk fully consumed
        st.store(xs);
        *reinterpret_cast<float4*>(&gs[threadIdx.x >> 6][(threadIdx.x & 63) * 4]) = gv;
        __syncthreads();
        if (k0 + kRouterKC < H) {
            st.load(x, row0, rows, H, k0 + kRouterKC);
            gv = *reinterpret_cast<const float4*>(gsrc + k0 + kRouterKC);
        }
        if (active) {
            // 16 blocks of 16 steps; the LDS reads of block i+1 are issued
            // before the FMAs of block i (ping-pong), pinned by sched_barrier
            float4 xa[4], ga[4], xb[4], gb[4];
            load_xg(xa, ga, 0);
#pragma unroll
            for (int blk = 0; blk < kRouterKC / 16; blk += 2) {
                load_xg(xb, gb, 16 * blk + 16);
                __builtin_amdgcn_sched_barrier(0);
                acc = fma16(acc, xa, ga);
                __builtin_amdgcn_sched_barrier(0);
                if (blk + 2 < kRouterKC / 16) load_xg(xa, ga, 16 * blk + 32);
                __builtin_amdgcn_sched_barrier(0);
                acc = fma16(acc, xb, gb);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    const int64_t row = row0 + lane;
    if (active && row < rows) logits[row * E + e] = acc;
}

// q = sign(l) * floorf(|l| / Q + 0.5f) * Q with every step rounded on its own
// (the _rn intrinsics keep the compiler from contracting the multiply into a
// later add).  src/layer.cu:72-77, src/tensor.cu:1300-1306.
__device__ inline float quantise(float l) {
    const float r = __fmul_rn(floorf(__fadd_rn(__fdiv_rn(fabsf(l), kRouterQuantum), 0.5f)),
                              kRouterQuantum);
    return l < 0.0f ? -r : r;
}

// One thread per token; one 64-thread workgroup per 64-token tile.  The
// token's E logits are loaded up front (independent loads, one round trip),
// then quantised and scanned twice.  Writes routes and the tile's per-expert
// histogram (popcounts of wave ballots: no atomics, deterministic).
template <int EMAX>
__global__ void __launch_bounds__(64)
k_route_top2(const float* __restrict__ logits, int64_t rows, int E, uint8_t* __restrict__ routes,
             uint32_t* __restrict__ tile_counts) {
    const int lane = threadIdx.x;
    const int64_t tile = blockIdx.x;
    const int64_t t = tile * kWave + lane;
    int first = 255, second = 255;
    if (t < rows) {
        float q[EMAX];
#pragma unroll
        for (int e = 0; e < EMAX; ++e) q[e] = e < E ? logits[t * E + e] : 0.0f;
#pragma unroll
        for (int e = 0; e < EMAX; ++e) q[e] = quantise(q[e]);
        // greedy scan: a later expert replaces the incumbent only when it is
        // larger by more than the tie epsilon (src/layer.cu:78-87)
        int best = -1;
        float bv = 0.0f;
#pragma unroll
        for (int e = 0; e < EMAX; ++e) {
            if (e < E && (best < 0 || q[e] > __fadd_rn(bv, kRouterTieEps))) { best = e; bv = q[e]; }
        }
        first = best;
        best = -1;
        bv = 0.0f;
#pragma unroll
        for (int e = 0; e < EMAX; ++e) {
            if (e < E && e != first && (best < 0 || q[e] > __fadd_rn(bv, kRouterTieEps))) { best = e; bv = q[e]; }
        }
        second = best;
        routes[2 * t] = static_cast<uint8_t>(first);
        routes[2 * t + 1] = static_cast<uint8_t>(second);
    }
    if (tile_counts) {
        uint32_t mine = 0;
        for (int e = 0; e < E; ++e) {
            const uint32_t c = __popcll(__ballot(first == e)) + __popcll(__ballot(second == e));
            if (lane == e) mine = c;
        }
        if (lane < E) tile_counts[tile * E + lane] = mine;
    }
}

}  // namespace

hipError_t launch_router_logits(const void* x, bool x_bf16, const float* gate, int64_t rows,
                                int hidden, int experts, float* logits, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hidden % kRouterKC != 0 || experts <= 0) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(ceil_div(rows, kWave)),
                    static_cast<unsigned>(ceil_div(experts, kRouterExpertsPerBlock)));
    if (x_bf16)
        hipLaunchKernelGGL(k_router_logits<true>, grid, dim3(256), 0, s, x, gate, rows, hidden,
                           experts, logits);
    else
        hipLaunchKernelGGL(k_router_logits<false>, grid, dim3(256), 0, s, x, gate, rows, hidden,
                           experts, logits);
    return hipGetLastError();
}

hipError_t launch_route_top2(const float* logits, int64_t rows, int experts, uint8_t* routes,
                             uint32_t* tile_counts, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (experts < 2 || experts > kMaxExperts) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(ceil_div(rows, kWave)));
    if (experts <= 16)
        hipLaunchKernelGGL(k_route_top2<16>, grid, dim3(64), 0, s, logits, rows, experts, routes, tile_counts);
    else
        hipLaunchKernelGGL(k_route_top2<kMaxExperts>, grid, dim3(64), 0, s, logits, rows, experts, routes,
                           tile_counts);
    return hipGetLastError();
}

}  // namespace aps
