// Token dispatch: stable counting sort of (token, slot) pairs by expert.
//
// Reference: k_moe_offsets_work (src/tensor.cu:1333-1374) scans counts on one
// thread, and k_moe_fill_stable (src/tensor.cu:1376-1418) runs one block per
// expert over ALL tokens, ranking with warp ballots.  The resulting order is
// fully determined: expert e's positions [offsets[e], offsets[e+1]) hold its
// tokens in ascending token order.
//
// gfx950 design: the routing kernel already produced a per-64-token-tile
// histogram (one word per tile and expert, one byte per 16-token quarter).
// Here each wave owns one tile:
//   1. lane e sums expert e's counts over all tiles (total) and over the
//      tiles before its own (prefix) -- a handful of L2-resident loads;
//   2. a wave scan over lanes turns totals into offsets;
//   3. for each expert, one 64-bit ballot + mbcnt-style popcount gives every
//      lane its stable rank inside the tile.
// Every (token, slot) is written exactly once, by the wave that owns the
// token, so the scatter is O(T) work instead of the reference's O(E*T).
#include "common.hpp"

namespace aps {
namespace {

// Fills n words with zero (a kernel rather than hipMemsetAsync, so the
// launch sequence stays safe to record into a HIP graph).
__global__ void k_zero_u32(uint32_t* __restrict__ p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

__global__ void __launch_bounds__(256)
k_tile_hist(const uint8_t* __restrict__ routes, int64_t rows, int E,
            uint32_t* __restrict__ tile_counts) {
    const int lane = threadIdx.x & 63;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t tile = t >> 6;
    const int64_t ntiles = (rows + kWave - 1) / kWave;
    int first = 255, second = 255;
    if (t < rows) {
        first = routes[2 * t];
        second = routes[2 * t + 1];
    }
    uint32_t mine = 0;
    for (int e = 0; e < E; ++e) {
        const uint32_t c = tile_quarter_counts(first, second, e);
        if (lane == e) mine = c;
    }
    if (tile < ntiles && lane < E) tile_counts[tile * E + lane] = mine;
}

__global__ void __launch_bounds__(256)
k_dispatch_scatter(const uint8_t* __restrict__ routes, const uint32_t* __restrict__ tile_counts,
                   int64_t rows, int E, uint32_t* __restrict__ counts,
                   uint32_t* __restrict__ offsets, uint32_t* __restrict__ assignment_rows,
                   uint32_t* __restrict__ route_positions) {
    const int lane = threadIdx.x & 63;
    const int64_t tile = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t ntiles = (rows + kWave - 1) / kWave;
    if (tile >= ntiles) return;  // wave-uniform

    // 1. per-expert totals and the prefix before this tile (lane = expert).
    //    Loads go out 32 tiles at a time (independent), so the wave waits a
    //    handful of L2 round trips rather than one per tile.
    uint32_t total = 0, before = 0;
    if (lane < E) {
        for (int64_t j0 = 0; j0 < ntiles; j0 += 32) {
            // unconditional loads (index clamped), so that all 32 are in
            // flight before the first use
            uint32_t c[32];
#pragma unroll
            for (int i = 0; i < 32; ++i) c[i] = tile_counts[(j0 + i < ntiles ? j0 + i : ntiles - 1) * E + lane];
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const uint32_t n = j0 + i < ntiles ? tile_word_total(c[i]) : 0u;
                total += n;
                before += j0 + i < tile ? n : 0u;
            }
        }
    }
    // 2. exclusive scan of totals over lanes 0..E-1
    uint32_t incl = total;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t v = __shfl_up(incl, d);
        if (lane >= d) incl += v;
    }
    const uint32_t excl = incl - total;
    const uint32_t base = excl + before;
    if (tile == 0 && lane < E) {
        counts[lane] = total;
        offsets[lane] = excl;
        if (lane == E - 1) offsets[E] = incl;
    }

    // 3. stable rank of each lane's token inside this tile, per expert
    const int64_t t = tile * kWave + lane;
    int first = 255, second = 255;
    if (t < rows) {
        first = routes[2 * t];
        second = routes[2 * t + 1];
    }
    const uint64_t below = (1ull << lane) - 1ull;
    uint32_t p0 = 0, p1 = 0;
    for (int e = 0; e < E; ++e) {
        const uint64_t m = __ballot(first == e || second == e);
        if (m == 0) continue;  // wave-uniform
        const uint32_t b = __shfl(base, e);
        const uint32_t r = static_cast<uint32_t>(__popcll(m & below));
        if (first == e) p0 = b + r;
        if (second == e) p1 = b + r;
    }
    if (t < rows) {
        assignment_rows[p0] = static_cast<uint32_t>(t);
        assignment_rows[p1] = static_cast<uint32_t>(t);
        route_positions[2 * t] = p0;
        route_positions[2 * t + 1] = p1;
    }
}

// Routing plan of a dense (single-expert) FFN: every row is position p = row
// of expert 0.
__global__ void k_dense_plan(uint32_t* __restrict__ offsets, uint32_t* __restrict__ rows_out, int64_t rows) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < rows) rows_out[i] = static_cast<uint32_t>(i);
    if (i == 0) {
        offsets[0] = 0u;
        offsets[1] = static_cast<uint32_t>(rows);
    }
}

}  // namespace

hipError_t launch_dense_plan(uint32_t* offsets, uint32_t* assignment_rows, int64_t rows, hipStream_t s) {
    const int64_t n = rows > 0 ? rows : 1;
    hipLaunchKernelGGL(k_dense_plan, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, s, offsets,
                       assignment_rows, rows);
    return hipGetLastError();
}

hipError_t launch_tile_hist(const uint8_t* routes, int64_t rows, int experts,
                            uint32_t* tile_counts, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_tile_hist, dim3(static_cast<unsigned>(ceil_div(rows, 256))), dim3(256),
                       0, s, routes, rows, experts, tile_counts);
    return hipGetLastError();
}

hipError_t launch_dispatch_scatter(const uint8_t* routes, const uint32_t* tile_counts,
                                   int64_t rows, int experts, uint32_t* counts,
                                   uint32_t* offsets, uint32_t* assignment_rows,
                                   uint32_t* route_positions, hipStream_t s) {
    if (experts <= 0 || experts > kMaxExperts) return hipErrorInvalidValue;
    if (rows <= 0) {
        // empty batch: counts and offsets are all zero
        hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(128), 0, s, counts, experts);
        hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(128), 0, s, offsets, experts + 1);
        return hipGetLastError();
    }
    const int64_t ntiles = ceil_div(rows, kWave);
    hipLaunchKernelGGL(k_dispatch_scatter, dim3(static_cast<unsigned>(ceil_div(ntiles, 4))),
                       dim3(256), 0, s, routes, tile_counts, rows, experts, counts, offsets,
                       assignment_rows, route_positions);
    return hipGetLastError();
}

}  // namespace aps
