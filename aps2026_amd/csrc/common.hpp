// Internal declarations shared by the gfx950 kernels and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace aps {

// Reference constants (include/config.h:22-23 of the reference).
constexpr float kRouterQuantum = 1.0e-3f;
constexpr float kRouterTieEps = 2.0e-2f;

constexpr int kWave = 64;           // CDNA wavefront width
constexpr int kTileTokens = 64;     // routing tile: one wave of tokens
constexpr int kMaxExperts = 64;     // routes are u8 and lane-indexed

// Grouped-GEMM row tile shared by the planner and the kernels.
constexpr int kUpBM = 128;          // w1||w3 kernel rows per tile
constexpr int kUpBN = 64;           // w1||w3 kernel intermediate cols per tile
constexpr int kDownBM = 128;        // w2 kernel rows per tile
constexpr int kDownBN = 128;        // w2 kernel hidden cols per tile
constexpr int kF32BM = 64;          // fp32 chain kernels rows per tile
constexpr int kF32BN = 64;          // fp32 chain kernels cols per tile

using bf16_t = uint16_t;            // raw bfloat16 bits in memory

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Upper bound on sum_e ceil(count_e / bm) over E experts with sum count_e = n.
__host__ __device__ inline int64_t max_row_tiles(int64_t n, int64_t bm, int64_t E) {
    return ceil_div(n, bm) + E;
}

// ---- launchers (defined in the .hip files) --------------------------------

hipError_t launch_router_logits(const void* x, bool x_bf16, const float* gate, int64_t rows,
                                int hidden, int experts, float* logits, hipStream_t s);
hipError_t launch_route_top2(const float* logits, int64_t rows, int experts, uint8_t* routes,
                             uint32_t* tile_counts, hipStream_t s);
hipError_t launch_tile_hist(const uint8_t* routes, int64_t rows, int experts,
                            uint32_t* tile_counts, hipStream_t s);
hipError_t launch_dispatch_scatter(const uint8_t* routes, const uint32_t* tile_counts,
                                   int64_t rows, int experts, uint32_t* counts,
                                   uint32_t* offsets, uint32_t* assignment_rows,
                                   uint32_t* route_positions, hipStream_t s);

// bf16 MFMA path.  w13 / w2 are packed tile images (see launch_pack_*):
// w13 [E][F/64][H/64][128][64], w2 [E][H/128][F/64][128][64]; act/y bf16.
hipError_t launch_ffn_up_bf16(const bf16_t* x, const uint32_t* offsets,
                              const uint32_t* assignment_rows, const bf16_t* w13,
                              bf16_t* act, int64_t rows, int hidden, int ffn, int experts,
                              hipStream_t s);
hipError_t launch_ffn_down_bf16(const bf16_t* act, const uint32_t* offsets, const bf16_t* w2,
                                bf16_t* y, int64_t rows, int hidden, int ffn, int experts,
                                hipStream_t s);

// fp32 FMA-chain path (reference accumulation order).  w1/w3 [E][F][H],
// w2 [E][H][F]; act/y are f32.
hipError_t launch_ffn_up_f32(const float* x, const uint32_t* offsets,
                             const uint32_t* assignment_rows, const float* w1,
                             const float* w3, float* act, int64_t rows, int hidden, int ffn,
                             int experts, hipStream_t s);
hipError_t launch_ffn_down_f32(const float* act, const uint32_t* offsets, const float* w2,
                               float* y, int64_t rows, int hidden, int ffn, int experts,
                               hipStream_t s);

hipError_t launch_combine(const void* y, bool y_bf16, const uint32_t* route_positions,
                          int64_t rows, int hidden, void* out, bool out_bf16, hipStream_t s);

// Weight packing helpers (registration time).
hipError_t launch_pack_w13_bf16(const void* const* w1, const void* const* w3, bool src_bf16,
                                bf16_t* dst, int experts, int ffn, int hidden, hipStream_t s);
hipError_t launch_pack_w2_bf16(const void* const* w2, bool src_bf16, bf16_t* dst, int experts, int ffn,
                               int hidden, hipStream_t s);

}  // namespace aps
