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
//   2. one pass over the experts, each expert's figures read from its lane
//      into scalar registers, scans the totals into offsets, and
//   3. in the same pass one 64-bit ballot + mbcnt-style popcount per expert
//      gives every lane its stable rank inside the tile.
// Every (token, slot) is written exactly once, by the wave that owns the
// token, so the scatter is O(T) work instead of the reference's O(E*T).
//
// SLOTS (the fused forward's folded combine): a second histogram counts the
// slot-0 routes alone, and the scatter also writes each expert's positions
// reordered by slot: list entries [offsets[e], slot1[e]) are the positions
// of the tokens whose first route is e, [slot1[e], offsets[e+1]) those whose
// second route is e, each in ascending token order (slot_rows = position,
// slot_tokens = token).  The positions themselves are the reference's.
#include "common.hpp"

namespace aps {
namespace {

// Fills n words with zero (a kernel rather than hipMemsetAsync, so the
// launch sequence stays safe to record into a HIP graph).
__global__ void k_zero_u32(uint32_t* __restrict__ p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// status (may be null): zeroed here, before k_dispatch_scatter counts the
// clamped route ids into it.
__global__ void __launch_bounds__(256)
k_tile_hist(const uint8_t* __restrict__ routes, int64_t rows, int E,
            uint32_t* __restrict__ tile_counts, uint32_t* __restrict__ status) {
    const int lane = threadIdx.x & 63;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t tile = t >> 6;
    const int64_t ntiles = (rows + kWave - 1) / kWave;
    if (status && t == 0) *status = 0u;
    int first = 255, second = 255;
    if (t < rows) {
        first = routes[2 * t];
        second = routes[2 * t + 1];
        clamp_routes(first, second, E);
    }
    uint32_t mine = 0;
    for (int e = 0; e < E; ++e) {
        const uint32_t c = tile_quarter_counts(first, second, e);
        if (lane == e) mine = c;
    }
    if (tile < ntiles && lane < E) tile_counts[tile * E + lane] = mine;
}

template <bool SLOTS>
__global__ void __launch_bounds__(256)
k_dispatch_scatter(const uint8_t* __restrict__ routes, const uint32_t* __restrict__ tile_counts,
                   int64_t rows, int E, uint32_t* __restrict__ counts,
                   uint32_t* __restrict__ offsets, uint32_t* __restrict__ assignment_rows,
                   uint32_t* __restrict__ route_positions, uint32_t* __restrict__ status,
                   const uint32_t* __restrict__ tile_counts0, uint32_t* __restrict__ slot1,
                   uint32_t* __restrict__ slot_rows, uint32_t* __restrict__ slot_tokens) {
    const int lane = threadIdx.x & 63;
    const int64_t tile = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t ntiles = (rows + kWave - 1) / kWave;

    // The lane's token's two routes (index clamped so that the loads are
    // unconditional), issued first: their latency overlaps the histogram
    // loads below.
    const int64_t t = tile * kWave + lane;
    const int64_t tc = t < rows ? t : rows - 1;
    const int r0 = routes[2 * tc], r1 = routes[2 * tc + 1];

    // 1. per-expert totals and the prefix before each of the workgroup's
    //    four tiles, with the histogram read once per workgroup: a load
    //    instruction covers tpl = 64 / E consecutive tiles (lane = tile
    //    offset x E + expert; tpl = 1 when E does not divide 64), and the
    //    four waves take every fourth group of tpl tiles.  Lanes of one
    //    expert are then summed with xor shuffles, the waves' sums in LDS.
    //    (Each wave reading the whole histogram, one narrow load per tile,
    //    was the kernel's main cost.)
    __shared__ uint32_t part[4][5][kMaxExperts];
    __shared__ uint32_t part0[SLOTS ? 4 : 1][5][kMaxExperts];   // slot-0 totals and prefixes
    const int wave = threadIdx.x >> 6;
    const int64_t tile0 = static_cast<int64_t>(blockIdx.x) * 4;  // the workgroup's first tile
    const int tpl = 64 % E == 0 ? 64 / E : 1;
    const int ex = lane % E;  // this lane's expert in the histogram loads
    const bool active = lane < tpl * E;
    // [0]: all routes, [1]: slot-0 routes (SLOTS)
    uint32_t tot[2] = {0, 0}, bef0[2] = {0, 0}, bef1[2] = {0, 0}, bef2[2] = {0, 0}, bef3[2] = {0, 0};
    // eight loads in flight per batch: unconditional (index clamped), used
    // only where the tile exists
    for (int64_t j0 = static_cast<int64_t>(wave) * tpl; j0 < ntiles; j0 += 32 * tpl) {
        uint32_t c[2][8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int64_t j = j0 + 4 * tpl * i + lane / E;
            const int64_t at = (j < ntiles ? j : ntiles - 1) * E + ex;
            c[0][i] = tile_counts[at];
            if constexpr (SLOTS) c[1][i] = tile_counts0[at];
        }
#pragma unroll
        for (int h = 0; h < (SLOTS ? 2 : 1); ++h)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int64_t j = j0 + 4 * tpl * i + lane / E;
                const uint32_t n = active && j < ntiles ? tile_word_total(c[h][i]) : 0u;
                tot[h] += n;
                bef0[h] += j < tile0 ? n : 0u;
                bef1[h] += j < tile0 + 1 ? n : 0u;
                bef2[h] += j < tile0 + 2 ? n : 0u;
                bef3[h] += j < tile0 + 3 ? n : 0u;
            }
    }
#pragma unroll
    for (int h = 0; h < (SLOTS ? 2 : 1); ++h)
        for (int d = E; d < 64 && tpl > 1; d <<= 1) {  // lanes e, e + E, e + 2E, ...
            tot[h] += __shfl_xor(tot[h], d);
            bef0[h] += __shfl_xor(bef0[h], d);
            bef1[h] += __shfl_xor(bef1[h], d);
            bef2[h] += __shfl_xor(bef2[h], d);
            bef3[h] += __shfl_xor(bef3[h], d);
        }
    if (lane < E) {
        part[wave][0][lane] = tot[0];
        part[wave][1][lane] = bef0[0];
        part[wave][2][lane] = bef1[0];
        part[wave][3][lane] = bef2[0];
        part[wave][4][lane] = bef3[0];
        if constexpr (SLOTS) {
            part0[wave][0][lane] = tot[1];
            part0[wave][1][lane] = bef0[1];
            part0[wave][2][lane] = bef1[1];
            part0[wave][3][lane] = bef2[1];
            part0[wave][4][lane] = bef3[1];
        }
    }
    __syncthreads();
    if (tile >= ntiles) return;  // wave-uniform, after the workgroup's barrier
    uint32_t total = 0, before = 0, total0 = 0, before0 = 0;
    if (lane < E) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            total += part[w][0][lane];
            before += part[w][1 + wave][lane];
            if constexpr (SLOTS) {
                total0 += part0[w][0][lane];
                before0 += part0[w][1 + wave][lane];
            }
        }
    }
    // 2./3. one pass over the experts, with expert e's figures read from
    //    lane e into scalar registers (v_readlane: no LDS round trip, unlike
    //    a shuffle): `run` is the exclusive scan of the totals, the offset
    //    of expert e; a ballot per slot and a popcount below the lane give
    //    each lane's stable rank inside the tile, the pairs of lower lanes
    //    first and slot 0 before slot 1.
    int first = 255, second = 255;
    if (t < rows) {
        first = r0;
        second = r1;
        const int bad = clamp_routes(first, second, E);
        if (status && bad) atomicAdd(status, static_cast<uint32_t>(bad));
    }
    const uint64_t below = (1ull << lane) - 1ull;
    uint32_t p0 = 0, p1 = 0, i0 = 0, i1 = 0, excl = 0, run = 0;
    for (int e = 0; e < E; ++e) {
        const uint32_t tot_e = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(total), e));
        if (lane == e) excl = run;
        const uint64_t m0 = __ballot(first == e), m1 = __ballot(second == e);
        if ((m0 | m1) != 0) {  // wave-uniform
            const uint32_t bef_e = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(before), e));
            const uint32_t b = run + bef_e;
            const uint32_t r = static_cast<uint32_t>(__popcll(m0 & below) + __popcll(m1 & below));
            if (first == e) p0 = b + r;
            if (second == e) p1 = b + r + (first == e ? 1u : 0u);
            if constexpr (SLOTS) {
                // list index of this tile's first slot-0 / slot-1 route of e
                const uint32_t tot0_e =
                    static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(total0), e));
                const uint32_t bef0_e =
                    static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(before0), e));
                const uint32_t l0 = run + bef0_e, l1 = run + tot0_e + (bef_e - bef0_e);
                if (first == e) i0 = l0 + static_cast<uint32_t>(__popcll(m0 & below));
                if (second == e) i1 = l1 + static_cast<uint32_t>(__popcll(m1 & below));
            }
        }
        run += tot_e;
    }
    if (tile == 0 && lane < E) {
        counts[lane] = total;
        offsets[lane] = excl;
        if (lane == E - 1) offsets[E] = run;
        if constexpr (SLOTS) slot1[lane] = excl + total0;
    }
    if (t < rows) {
        assignment_rows[p0] = static_cast<uint32_t>(t);
        assignment_rows[p1] = static_cast<uint32_t>(t);
        route_positions[2 * t] = p0;
        route_positions[2 * t + 1] = p1;
        if constexpr (SLOTS) {
            // in range whenever the slot-0 histogram matches the routes
            const uint32_t A = static_cast<uint32_t>(2 * rows);
            if (i0 < A) {
                slot_rows[i0] = p0;
                slot_tokens[i0] = static_cast<uint32_t>(t);
            }
            if (i1 < A) {
                slot_rows[i1] = p1;
                slot_tokens[i1] = static_cast<uint32_t>(t);
            }
        }
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
                            uint32_t* tile_counts, uint32_t* status, hipStream_t s) {
    if (rows <= 0) {
        if (status) hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(64), 0, s, status, 1);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_tile_hist, dim3(static_cast<unsigned>(ceil_div(rows, 256))), dim3(256),
                       0, s, routes, rows, experts, tile_counts, status);
    return hipGetLastError();
}

hipError_t launch_dispatch_scatter(const uint8_t* routes, const uint32_t* tile_counts,
                                   int64_t rows, int experts, uint32_t* counts,
                                   uint32_t* offsets, uint32_t* assignment_rows,
                                   uint32_t* route_positions, uint32_t* status, hipStream_t s,
                                   const uint32_t* tile_counts0, uint32_t* slot1, uint32_t* slot_rows,
                                   uint32_t* slot_tokens) {
    if (experts <= 0 || experts > kMaxExperts) return hipErrorInvalidValue;
    const bool slots = tile_counts0 != nullptr;
    if (slots && (!slot1 || !slot_rows || !slot_tokens)) return hipErrorInvalidValue;
    if (rows <= 0) {
        // empty batch: counts and offsets are all zero
        hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(128), 0, s, counts, experts);
        hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(128), 0, s, offsets, experts + 1);
        if (slots) hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(128), 0, s, slot1, experts);
        return hipGetLastError();
    }
    const int64_t ntiles = ceil_div(rows, kWave);
    const dim3 grid(static_cast<unsigned>(ceil_div(ntiles, 4)));
    if (slots)
        hipLaunchKernelGGL(k_dispatch_scatter<true>, grid, dim3(256), 0, s, routes, tile_counts, rows, experts,
                           counts, offsets, assignment_rows, route_positions, status, tile_counts0, slot1,
                           slot_rows, slot_tokens);
    else
        hipLaunchKernelGGL(k_dispatch_scatter<false>, grid, dim3(256), 0, s, routes, tile_counts, rows, experts,
                           counts, offsets, assignment_rows, route_positions, status, nullptr, nullptr,
                           nullptr, nullptr);
    return hipGetLastError();
}

}  // namespace aps
