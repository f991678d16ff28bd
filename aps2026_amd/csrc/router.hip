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
//    each lane reads its own row with ds_read_b128 (row pitch 260 floats
//    keeps the eight lanes of each LDS phase on distinct banks).
//  * gate: the value of step k is the same for the whole wave.  Each lane of
//    a 16-lane DPP row holds 16 consecutive gate values spread over the row
//    (lane j of the row holds gate[k0 + 16c + j] in register c), and step
//    k0 + 16c + j reads it with a DPP row_newbcast:j broadcast.  This keeps
//    the gate out of SGPRs (scalar loads return out of order, which would
//    force a full lgkmcnt wait on every prefetch) and costs one VMEM dword
//    per lane per 16 steps.
//  * x and gate for the next 64 steps are in flight while the current 64
//    FMAs run (explicit ping-pong), so latency hides even at one wave per
//    SIMD, which is the occupancy the chain count gives at T = 4096.
// Four waves (four experts) share an x tile; the grid is [token tiles] x
// [E/4], and with tiles % 8 == 0 the four expert groups of a tile land on one
// XCD (blocks are dealt round-robin over the 8 XCDs), so x is fetched from
// HBM once per XCD L2.  The next 256-wide x chunk is prefetched into
// registers while the current one is consumed.
#include "common.hpp"

namespace aps {
namespace {

constexpr int kRouterKC = 256;              // k per LDS chunk
constexpr int kRouterPitch = kRouterKC + 4; // floats per LDS row
constexpr int kRouterExpertsPerBlock = 4;   // one wave per expert

// Loads one 64 x kc chunk of x into registers (8 values per 16-byte piece).
template <bool XBF16>
struct XStage;

template <>
struct XStage<true> {
    // 64 rows * 256 bf16 = 2048 pieces of 8 bf16 -> 8 per thread
    static constexpr int kPieces = 8;
    uint4 v[kPieces];
    __device__ void load(const bf16_t* x, int64_t row0, int64_t rows, int H, int k0, int kc) {
#pragma unroll
        for (int j = 0; j < kPieces; ++j) {
            const int p = threadIdx.x + j * 256;
            const int r = p >> 5;           // 32 pieces per 256-wide row
            const int c = (p & 31) * 8;
            const int64_t row = row0 + r;
            if (c < kc && row < rows)
                v[j] = *reinterpret_cast<const uint4*>(x + row * H + k0 + c);
            else
                v[j] = make_uint4(0, 0, 0, 0);
        }
    }
    __device__ void store(float* xs) const {
#pragma unroll
        for (int j = 0; j < kPieces; ++j) {
            const int p = threadIdx.x + j * 256;
            const int r = p >> 5;
            const int c = (p & 31) * 8;
            float* d = xs + r * kRouterPitch + c;
            const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
            float f[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f[2 * i] = __uint_as_float(w[i] << 16);
                f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
            }
            *reinterpret_cast<float4*>(d) = make_float4(f[0], f[1], f[2], f[3]);
            *reinterpret_cast<float4*>(d + 4) = make_float4(f[4], f[5], f[6], f[7]);
        }
    }
};

template <>
struct XStage<false> {
    // 64 rows * 256 f32 = 4096 pieces of 4 floats -> 16 per thread
    static constexpr int kPieces = 16;
    float4 v[kPieces];
    __device__ void load(const float* x, int64_t row0, int64_t rows, int H, int k0, int kc) {
#pragma unroll
        for (int j = 0; j < kPieces; ++j) {
            const int p = threadIdx.x + j * 256;
            const int r = p >> 6;           // 64 pieces per 256-wide row
            const int c = (p & 63) * 4;
            const int64_t row = row0 + r;
            if (c < kc && row < rows)
                v[j] = *reinterpret_cast<const float4*>(x + row * H + k0 + c);
            else
                v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    __device__ void store(float* xs) const {
#pragma unroll
        for (int j = 0; j < kPieces; ++j) {
            const int p = threadIdx.x + j * 256;
            const int r = p >> 6;
            const int c = (p & 63) * 4;
            *reinterpret_cast<float4*>(xs + r * kRouterPitch + c) = v[j];
        }
    }
};

// 16 chain steps acc = fma(g_k, x_k, acc), k = 0..15 in order, where g_k is
// lane k of this lane's 16-lane DPP row (row_newbcast:k folded into
// v_fmac_f32_dpp, one fused multiply-add per step) and x_k the lane's own
// value.  The leading s_nop covers the DPP read-after-VALU-write hazard on
// `g` (two wait states); `g` is not written inside the block.
__device__ inline float fma16_rowbcast(float acc, float g, const float4& a, const float4& b,
                                       const float4& c, const float4& d) {
    asm("s_nop 1\n\t"
        "v_fmac_f32_dpp %0, %1, %2 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %3 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %4 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %5 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %6 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %7 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %8 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %9 row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %10 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %11 row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %12 row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %13 row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %14 row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %15 row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %16 row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"
        "v_fmac_f32_dpp %0, %1, %17 row_newbcast:15 row_mask:0xf bank_mask:0xf\n\t"
        : "+v"(acc)
        : "v"(g), "v"(a.x), "v"(a.y), "v"(a.z), "v"(a.w), "v"(b.x), "v"(b.y), "v"(b.z), "v"(b.w),
          "v"(c.x), "v"(c.y), "v"(c.z), "v"(c.w), "v"(d.x), "v"(d.y), "v"(d.z), "v"(d.w));
    return acc;
}

template <bool XBF16>
__global__ void __launch_bounds__(256, 2)
k_router_logits(const void* __restrict__ xv, const float* __restrict__ gate, int64_t rows,
                int H, int E, float* __restrict__ logits) {
    using XT = typename std::conditional<XBF16, bf16_t, float>::type;
    const XT* __restrict__ x = static_cast<const XT*>(xv);
    __shared__ __align__(16) float xs[kWave * kRouterPitch];

    const int lane = threadIdx.x & 63;
    const int e = blockIdx.y * kRouterExpertsPerBlock + (threadIdx.x >> 6);
    const bool active = e < E;  // wave-uniform
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kWave;
    const float* __restrict__ gsrc = gate + static_cast<int64_t>(active ? e : 0) * H + (lane & 15);
    const float* xrow = xs + lane * kRouterPitch;

    auto load_x = [&](float4 (&d)[4], int kk) {
#pragma unroll
        for (int i = 0; i < 4; ++i) d[i] = *reinterpret_cast<const float4*>(xrow + kk + 4 * i);
    };
    auto load_g = [&](float (&d)[4], int k) {
#pragma unroll
        for (int c = 0; c < 4; ++c) d[c] = gsrc[k + 16 * c];
    };

    // Issue order matters: VMEM returns in order, so the gate loads of a
    // chunk are issued at the end of the previous chunk (after that chunk's
    // x staging loads were consumed), never behind the next staging loads.
    XStage<XBF16> st;
    float g[4][4];
    st.load(x, row0, rows, H, 0, kRouterKC);
    if (active) {
#pragma unroll
        for (int q = 0; q < 4; ++q) load_g(g[q], 64 * q);
    }
    float acc = 0.0f;
    for (int k0 = 0; k0 < H; k0 += kRouterKC) {
        __syncthreads();  // previous chunk fully consumed
        st.store(xs);
        __syncthreads();
        const bool more = k0 + kRouterKC < H;
        if (more) st.load(x, row0, rows, H, k0 + kRouterKC, kRouterKC);
        if (active) {
            // 16 blocks of 16 steps.  The LDS reads of block i+1 are issued
            // before the FMAs of block i (ping-pong between xa and xb); the
            // sched_barriers pin that order against the scheduler, which
            // would otherwise sink each read next to its use.
            float4 xa[4], xb[4];
            load_x(xa, 0);
#pragma unroll
            for (int blk = 0; blk < kRouterKC / 16; blk += 2) {
                load_x(xb, 16 * blk + 16);
                __builtin_amdgcn_sched_barrier(0);
                acc = fma16_rowbcast(acc, g[blk >> 2][blk & 3], xa[0], xa[1], xa[2], xa[3]);
                __builtin_amdgcn_sched_barrier(0);
                if (blk + 2 < kRouterKC / 16) load_x(xa, 16 * blk + 32);
                __builtin_amdgcn_sched_barrier(0);
                acc = fma16_rowbcast(acc, g[(blk + 1) >> 2][(blk + 1) & 3], xb[0], xb[1], xb[2], xb[3]);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (more) {
#pragma unroll
                for (int q = 0; q < 4; ++q) load_g(g[q], k0 + kRouterKC + 64 * q);
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

// One thread per token; one wave per 64-token tile.  Writes routes and the
// tile's per-expert histogram (popcounts of wave ballots: no atomics, so the
// histogram is deterministic).
__global__ void __launch_bounds__(256)
k_route_top2(const float* __restrict__ logits, int64_t rows, int E, uint8_t* __restrict__ routes,
             uint32_t* __restrict__ tile_counts) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    int first = 255, second = 255;
    if (t < rows) {
        const float* l = logits + t * E;
        // greedy scan: a later expert replaces the incumbent only when it is
        // larger by more than the tie epsilon (src/layer.cu:78-87)
        int best = -1;
        float bv = 0.0f;
        for (int e = 0; e < E; ++e) {
            const float q = quantise(l[e]);
            if (best < 0 || q > __fadd_rn(bv, kRouterTieEps)) { best = e; bv = q; }
        }
        first = best;
        best = -1;
        bv = 0.0f;
        for (int e = 0; e < E; ++e) {
            if (e == first) continue;
            const float q = quantise(l[e]);
            if (best < 0 || q > __fadd_rn(bv, kRouterTieEps)) { best = e; bv = q; }
        }
        second = best;
        routes[2 * t] = static_cast<uint8_t>(first);
        routes[2 * t + 1] = static_cast<uint8_t>(second);
    }
    if (tile_counts) {
        const int lane = threadIdx.x & 63;
        const int64_t tile = t >> 6;
        const int64_t ntiles = (rows + kWave - 1) / kWave;
        uint32_t mine = 0;
        for (int e = 0; e < E; ++e) {
            const uint32_t c = __popcll(__ballot(first == e)) + __popcll(__ballot(second == e));
            if (lane == e) mine = c;
        }
        if (tile < ntiles && lane < E) tile_counts[tile * E + lane] = mine;
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
    hipLaunchKernelGGL(k_route_top2, dim3(static_cast<unsigned>(ceil_div(rows, 256))), dim3(256),
                       0, s, logits, rows, experts, routes, tile_counts);
    return hipGetLastError();
}

}  // namespace aps
