// Internal declarations shared by the gfx950 kernels and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

namespace aps {

// Reference constants (include/config.h:22-23 of the reference).
constexpr float kRouterQuantum = 1.0e-3f;
constexpr float kRouterTieEps = 2.0e-2f;

constexpr int kWave = 64;           // CDNA wavefront width
constexpr int kTileTokens = 64;     // routing tile: one wave of tokens
constexpr int kMaxExperts = 64;     // routes are u8 and lane-indexed

constexpr int kF32BM = 64;          // fp32 chain kernels rows per tile
constexpr int kF32BN = 64;          // fp32 chain kernels cols per tile

using bf16_t = uint16_t;            // raw bfloat16 bits in memory

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// q = sign(l) * floorf(|l| / Q + 0.5f) * Q with every step rounded on its own
// (the _rn intrinsics keep the compiler from contracting the multiply into a
// later add).  Reference src/layer.cu:72-77, src/tensor.cu:1300-1306.
__device__ inline float route_quantise(float l) {
    const float r = __fmul_rn(floorf(__fadd_rn(__fdiv_rn(fabsf(l), kRouterQuantum), 0.5f)), kRouterQuantum);
    return l < 0.0f ? -r : r;
}

// Greedy top-2 over the quantised logits q[0..E-1]: a later expert replaces
// the incumbent only when it is larger by more than the tie epsilon
// (reference src/layer.cu:78-87, src/tensor.cu:1307-1330).
template <int EMAX>
__device__ inline void route_greedy_top2(const float (&q)[EMAX], int E, int& first, int& second) {
    int best = -1;
    float bv = 0.0f;
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
        if (e < E && (best < 0 || q[e] > __fadd_rn(bv, kRouterTieEps))) { best = e; bv = q[e]; }
    first = best;
    best = -1;
    bv = 0.0f;
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
        if (e < E && e != first && (best < 0 || q[e] > __fadd_rn(bv, kRouterTieEps))) { best = e; bv = q[e]; }
    second = best;
}

// Tile histogram word of expert e for the 64-token tile of this wave: byte q
// counts the routes to e of tokens 16q .. 16q+15 (at most 16 each), so a word
// sums to the tile's count with (w * 0x01010101) >> 24.  The router writes the
// bytes one 16-token workgroup at a time.
__device__ inline uint32_t tile_quarter_counts(int first, int second, int e) {
    const uint64_t m0 = __ballot(first == e), m1 = __ballot(second == e);
    uint32_t word = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint64_t qm = 0xFFFFull << (16 * q);
        word |= static_cast<uint32_t>(__popcll(m0 & qm) + __popcll(m1 & qm)) << (8 * q);
    }
    return word;
}
__host__ __device__ inline uint32_t tile_word_total(uint32_t w) { return (w * 0x01010101u) >> 24; }

// The reference's combine of a token's two expert outputs (k_moe_combine,
// src/tensor.cu:1968-1988): value = 0, then value += 0.5 a, value += 0.5 b,
// each step rounded.  0.5 v is exact, so the order of a and b changes no
// bit; the leading 0 turns a -0 first term into +0 (two -0 terms give +0).
__device__ inline float moe_combine2(float a, float b) {
    return __fadd_rn(__fadd_rn(0.0f, __fmul_rn(0.5f, a)), __fmul_rn(0.5f, b));
}

// ---- fp8 e4m3 row quantisation (the library's fp8 format) ------------------
// scale = amax(|row|) / 448 (1 if the row is all zero), code = e4m3(v / scale)
// with nearest-even rounding, saturating at +-448 (OCP "e4m3fn").  Shared by
// the row quantiser and the router's x quantisation, so that both give the
// same bits.
typedef uint32_t e4m3_words_t __attribute__((ext_vector_type(4)));  // 8 bf16 values
constexpr float kE4m3Max = 448.0f;

// e4m3 codes of two fp32 values in bytes 2 kHi, 2 kHi + 1 of `old`: gfx950's
// v_cvt_pk_fp8_f32 (OCP e4m3, round to nearest even).  For every fp32 |v| <=
// 464 (a row quotient is at most 448 plus rounding) it equals the encoder
// "keep 3 mantissa bits, ties to even; subnormal grid 2^-9; saturate at 448"
// bit for bit, -0 and subnormals included: 2.28e9 values checked on the GPU.
template <bool kHi>
__device__ inline uint32_t e4m3_pack2(float a, float b, uint32_t old) {
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, static_cast<int>(old), kHi));
}

// v / sc as IEEE division rounds it, for its e4m3 code, from the row's
// reciprocal r = RN(1 / sc): q0 = RN(v r), then one Markstein correction
// q = RN(q0 + RN(v - q0 sc) r) with both steps fused (the residual is exact
// while it stays normal), given v's sign so that -0 stays -0.  Valid for
// sc >= 2^-89: then a value whose residual could underflow has a quotient
// below 2^-10, whose code is +-0 either way.  For every bf16 amax >= 448 *
// 2^-89 and every bf16 |v| <= amax the code equals that of the IEEE quotient
// (1.07e9 pairs, tests/cpp/quotient_check.c; without the correction 58,276
// of them differ).  A multiply and two FMAs replace a ten-instruction
// division per value.
constexpr float kMinFastScale = 0x1p-89f;
__device__ inline float e4m3_quotient(float v, float sc, float r) {
    const float q0 = __fmul_rn(v, r);
    return copysignf(__fmaf_rn(__fmaf_rn(-q0, sc, v), r, q0), v);
}
__device__ inline float bf16w_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float bf16w_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// The running |v| maximum of a row over the 8 bf16 values of w (fmaxf
// ignores NaN; the maximum does not depend on the order of the values).
__device__ inline float e4m3_amax8(float amax, const e4m3_words_t& w) {
#pragma unroll
    for (int k = 0; k < 4; ++k) amax = fmaxf(amax, fmaxf(fabsf(bf16w_lo(w[k])), fabsf(bf16w_hi(w[k]))));
    return amax;
}
// The row's scale from its amax.
__device__ inline float e4m3_row_scale(float amax) {
    const float sc = __fdiv_rn(amax, kE4m3Max);
    return sc > 0.0f ? sc : 1.0f;
}

// Codes of the 8 bf16 values of one 16-byte chunk, as two words.
template <bool kFast>
__device__ inline void e4m3_chunk_codes(const e4m3_words_t& w, float sc, float rc, uint32_t& lo, uint32_t& hi) {
    float q[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float a = bf16w_lo(w[k]), b = bf16w_hi(w[k]);
        q[2 * k] = kFast ? e4m3_quotient(a, sc, rc) : __fdiv_rn(a, sc);
        q[2 * k + 1] = kFast ? e4m3_quotient(b, sc, rc) : __fdiv_rn(b, sc);
    }
    lo = e4m3_pack2<true>(q[2], q[3], e4m3_pack2<false>(q[0], q[1], 0u));
    hi = e4m3_pack2<true>(q[6], q[7], e4m3_pack2<false>(q[4], q[5], 0u));
}

// Caller-supplied routes (aps_moe_dispatch) are made memory-safe before they
// are counted or ranked: an expert id >= E is clamped to E - 1 (and reported
// by the caller-visible counter), a token whose two slots name the same
// expert keeps both -- it takes two consecutive positions of that expert,
// slot 0 first, as a stable sort of the (token, slot) pairs gives.  Routes
// the router writes are always two distinct ids < E, which this leaves
// unchanged.  Returns the number of clamped ids (0..2).
__device__ inline int clamp_routes(int& r0, int& r1, int E) {
    int bad = 0;
    if (r0 >= E) { r0 = E - 1; ++bad; }
    if (r1 >= E) { r1 = E - 1; ++bad; }
    return bad;
}

// Upper bound on sum_e ceil(count_e / bm) over E experts with sum count_e = n.
__host__ __device__ inline int64_t max_row_tiles(int64_t n, int64_t bm, int64_t E) {
    return ceil_div(n, bm) + E;
}

// Row-tile lookup shared by the grouped GEMMs.  Row tiles run over experts
// in order, expert e owning ceil(count_e / bm) tiles of bm positions.  One
// vector load brings offsets[0..E] into lanes 0..E, a wave prefix scan turns
// per-expert tile counts into running totals, and a ballot finds the expert
// of `tile` -- one memory round trip instead of a dependent chain of scalar
// loads.  Every output is wave-uniform.  E <= 64.
struct RowTile {
    int expert;
    uint32_t m0, end;
};

__device__ inline int wave_tile_scan(const uint32_t* __restrict__ offsets, int E, int bm, uint32_t& lo,
                                     uint32_t& hi, int& incl) {
    const int lane = threadIdx.x & 63;
    lo = lane < E ? offsets[lane] : 0u;
    hi = __shfl_down(lo, 1);
    if (lane == E - 1) hi = offsets[E];
    const int nt = lane < E ? static_cast<int>((hi - lo + bm - 1) / bm) : 0;
    incl = nt;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int v = __shfl_up(incl, d);
        if (lane >= d) incl += v;
    }
    return __shfl(incl, 63);  // total row tiles
}

__device__ inline RowTile wave_find_tile(int tile, int bm, uint32_t lo, uint32_t hi, int incl, int E) {
    const int lane = threadIdx.x & 63;
    const uint64_t m = __ballot(lane < E && incl > tile);
    const int e = __ffsll(static_cast<unsigned long long>(m)) - 1;
    const int start = __shfl(incl, e > 0 ? e - 1 : 0);
    const int before = e > 0 ? start : 0;
    RowTile r;
    r.expert = e;
    r.m0 = __shfl(lo, e) + static_cast<uint32_t>(tile - before) * bm;
    r.end = __shfl(hi, e);
    return r;
}

// ---- launchers (defined in the .hip files) --------------------------------

// Router GEMM; with routes != nullptr also the top-2 routes and the tile
// histogram (tile_counts), in the same kernel, and with tile_counts0 !=
// nullptr the histogram of slot-0 routes alone; with x_copy != nullptr (fp32
// x only) also the bf16 copy of x [rows][hidden]; with xq, xq_scale !=
// nullptr (bf16 x, router_quantises_x) also the e4m3 codes of x [rows][hidden]
// and the row scales [rows], equal to launch_quant_rows_e4m3's.
int num_cus();  // compute units of the current device
bool router_quantises_x(int hidden, int experts);
hipError_t launch_router(const void* x, bool x_bf16, const float* gate, int64_t rows, int hidden,
                         int experts, float* logits, uint8_t* routes, uint32_t* tile_counts,
                         uint32_t* tile_counts0, bf16_t* x_copy, uint8_t* xq, float* xq_scale, hipStream_t s);
hipError_t launch_route_top2(const float* logits, int64_t rows, int experts, uint8_t* routes,
                             uint32_t* tile_counts, hipStream_t s);
// status (may be null): one u32 that counts the route ids >= experts the
// dispatch clamped (zeroed by launch_tile_hist, added to by the scatter).
hipError_t launch_tile_hist(const uint8_t* routes, int64_t rows, int experts,
                            uint32_t* tile_counts, uint32_t* status, hipStream_t s);
// Decoder-layer LayerNorm (residual == nullptr: plain; else x += residual
// in place first).  hidden % 256 == 0.
// Row gather out[i] = x[rows[i]] (fp32); rows past x_rows give zero rows.
hipError_t launch_gather_rows(const float* x, int64_t x_rows, int64_t hidden, const uint32_t* rows, int64_t count,
                              float* out, hipStream_t s);

// Prefix-trie deduplication of a packed prompt batch (host code).  Returns 0,
// 1 for the reference's std::invalid_argument conditions or 2 for other
// invalid arguments, with a message in err.
int prefix_dedup(const int32_t* ids, const int64_t* seq_offsets, int64_t batch, int64_t vocab, int64_t max_positions,
                 uint32_t* token_node, uint32_t* node_token, uint32_t* node_depth, uint32_t* node_anc,
                 int64_t anc_stride, int64_t* nodes_out, std::string& err);
// The ancestor table [nodes][stride] of a trie from its parent, depth and
// run-start arrays (device memory); see prefix.hip.
hipError_t launch_prefix_ancestors(const uint32_t* parent, const uint32_t* depth, const uint32_t* run_start,
                                   int64_t nodes, int64_t stride, uint32_t* anc, hipStream_t s);

// RoPE in place on x [rows][heads][head_dim] at each row's position (pairs
// j, j + head_dim / 2); rows whose position is >= max_seq are left as they are.
hipError_t launch_rope_tree(float* x, const uint32_t* row_pos, int64_t rows, int heads, int head_dim,
                            const float* cosv, const float* sinv, int64_t max_seq, hipStream_t s);

// GQA-4 tree attention, head_dim 128 (the reference kernel's arithmetic).
// A workgroup keeps 20 bytes of LDS per key of its window (four scores and
// the key's row index) next to 2 KB of its own: windows up to kAttnMaxWindow
// keys fit gfx950's 160 KB of LDS per workgroup.
constexpr int kAttnMaxWindow = 7936;
hipError_t launch_attention_tree(const float* q, const float* k, const float* v, float* out, const uint32_t* row_pos,
                                 const uint32_t* anc, int64_t anc_stride, int64_t rows, int q_heads, int kv_heads,
                                 int head_dim, int window_max, bool packed, hipStream_t s);
// Packed-sequence attention for any head layout (q_heads % kv_heads == 0,
// head_dim <= 128): the reference's generic kernel's arithmetic.
hipError_t launch_attention_any(const float* q, const float* k, const float* v, float* out, const uint32_t* seg_offset,
                                const uint32_t* seg_pos, int64_t max_seq, int64_t rows, int q_heads, int kv_heads,
                                int head_dim, int window_max, hipStream_t s);

// Elementwise fp32 ops (reference k_add, k_add_bias, k_silu_mul, zero_gpu).
hipError_t launch_add_inplace(float* a, const float* b, int64_t n, hipStream_t s);
hipError_t launch_add_bias(float* a, const float* bias, int64_t n, int h, hipStream_t s);
hipError_t launch_silu_mul(const float* g, const float* u, float* out, int64_t n, hipStream_t s);
hipError_t launch_zero(float* x, int64_t n, hipStream_t s);

// Split-bf16 Linear (the reference's optional tensor-core path): W packed
// into hi / lo bf16 tile images, x split into hi / lo bf16 rows, products
// hi.hi + hi.lo + lo.hi (+ lo.lo) on the bf16 MFMA (in_f % 64 == 0).
int64_t linear_tc_packed_elems(int out_f, int in_f);
hipError_t launch_linear_tc_prepare(const float* w, int out_f, int in_f, uint16_t* packed, hipStream_t s);
hipError_t launch_split_bf16(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, hipStream_t s);
hipError_t launch_linear_tc(const uint16_t* xhi, const uint16_t* xlo, const uint16_t* packed, const float* bias,
                            float* y, int64_t rows, int in_f, int out_f, bool all_terms, hipStream_t s);
// up to three outputs of one split input in one launch
hipError_t launch_linear_tc_multi(const uint16_t* xhi, const uint16_t* xlo, int count, const uint16_t* const* packed,
                                  const float* const* bias, float* const* y, const int* out_f, int64_t rows, int in_f,
                                  bool all_terms, hipStream_t s);

// y = x w^T (+ bias): fp32 FMA chain over k ascending per output, bias added
// once (in_f % 16 == 0, out_f % 4 == 0).
// fp32 Linear on the K = 1 fp32 MFMA (same bits as the FMA chain); shapes
// with in_f % 32 == 0
bool linear_mfma_fits(int64_t rows, int in_f, int out_f);
hipError_t launch_linear_mfma_f32(const float* x, const float* w, const float* bias, float* y, int64_t rows,
                                  int in_f, int out_f, hipStream_t s);
// count (1..3) outputs of one x in one grid, every shape linear_mfma_fits
hipError_t launch_linear_mfma_multi(const float* x, int64_t rows, int in_f, int count, const float* const* w,
                                    const float* const* bias, float* const* y, const int* out_f, hipStream_t s);
hipError_t launch_linear_f32(const float* x, const float* w, const float* bias, float* y, int64_t rows, int in_f,
                             int out_f, hipStream_t s);
// the same chains for any in_f, out_f and 4-byte alignment (SIMT, scalar loads)
hipError_t launch_linear_any_f32(const float* x, const float* w, const float* bias, float* y, int64_t rows, int in_f,
                                 int out_f, hipStream_t s);

hipError_t launch_layer_norm(float* x, const float* residual, const float* weight, const float* bias, float* y,
                             int64_t rows, int hidden, float eps, hipStream_t s);
// With tile_counts0 (the slot-0 histogram) also the slot-ordered lists:
// slot1[e] = offsets[e] + (slot-0 routes of e); slot_rows / slot_tokens
// [2 rows] = position / token of list entry i (see dispatch.hip).
hipError_t launch_dispatch_scatter(const uint8_t* routes, const uint32_t* tile_counts,
                                   int64_t rows, int experts, uint32_t* counts,
                                   uint32_t* offsets, uint32_t* assignment_rows,
                                   uint32_t* route_positions, uint32_t* status, hipStream_t s,
                                   const uint32_t* tile_counts0 = nullptr, uint32_t* slot1 = nullptr,
                                   uint32_t* slot_rows = nullptr, uint32_t* slot_tokens = nullptr);

// bf16 MFMA path.  w13 / w2 are packed tile images (see launch_pack_*):
// w13 [E][F/64][H/64][128][64], w2 [E][H/128][F/64][128][64]; act/y bf16.
// The fp8 path's images are 128 x 128 bytes: w13 [E][F/64][H/128][128][128],
// w2 [E][H/128][Kp/128][128][128] (Kp = F rounded up to 128, zero padded).
hipError_t launch_ffn_up_bf16(const bf16_t* x, const uint32_t* offsets,
                              const uint32_t* assignment_rows, const bf16_t* w13,
                              bf16_t* act, int64_t rows, int hidden, int ffn, int experts,
                              hipStream_t s);
hipError_t launch_ffn_down_bf16(const bf16_t* act, const uint32_t* offsets, const bf16_t* w2,
                                bf16_t* y, int64_t rows, int hidden, int ffn, int experts,
                                hipStream_t s);

// fp8 e4m3 MFMA path.  xq [rows][H] codes with x_scale [rows]; act is bf16
// [A][F]; actq [A][Kp] codes with act_scale [A]; w*_scale per output
// channel ([E][F] for w1/w3, [E][H] for w2); y bf16.
hipError_t launch_ffn_up_fp8(const uint8_t* xq, const float* x_scale, const uint32_t* offsets,
                             const uint32_t* assignment_rows, const uint8_t* w13, const float* w1_scale,
                             const float* w3_scale, bf16_t* act, int64_t rows, int hidden, int ffn,
                             int experts, hipStream_t s);
hipError_t launch_ffn_down_fp8(const uint8_t* actq, const float* act_scale, const uint32_t* offsets,
                               const uint8_t* w2, const float* w2_scale, bf16_t* y, int64_t rows, int hidden,
                               int ffn, int experts, hipStream_t s);
// The fp8 w2 GEMM with the combine folded in (two launches over the
// dispatch's slot-ordered lists): slot-0 rows to ya [rows][hidden] bf16 by
// token, then slot-1 rows combined with them into out [rows][hidden] bf16.
// ffn_down_fold_fits: the shapes it serves.
bool ffn_down_fold_fits(int64_t rows, int hidden, int ffn);
hipError_t launch_ffn_down_fold_fp8(const uint8_t* actq, const float* act_scale, const uint32_t* offsets,
                                    const uint32_t* slot1, const uint32_t* slot_rows, const uint32_t* slot_tokens,
                                    const uint8_t* w2, const float* w2_scale, bf16_t* ya, bf16_t* out,
                                    int64_t rows, int hidden, int ffn, int experts, hipStream_t s);
// Per-row e4m3 quantisation of bf16 rows (n values, row strides in
// elements / bytes; codes zero-padded to dst_stride).
hipError_t launch_quant_rows_e4m3(const bf16_t* src, int64_t src_stride, int n, uint8_t* dst, int64_t dst_stride,
                                  float* scale, int64_t rows, hipStream_t s);
hipError_t launch_pack_w13_e4m3(const void* const* w1, const void* const* w3, uint8_t* dst, int experts, int ffn,
                                int hidden, hipStream_t s);
hipError_t launch_pack_w2_e4m3(const void* const* w2, uint8_t* dst, int experts, int ffn, int hidden,
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

// Dense (single-expert) plan: offsets = {0, rows}, assignment_rows[i] = i.
hipError_t launch_dense_plan(uint32_t* offsets, uint32_t* assignment_rows, int64_t rows, hipStream_t s);

// dst = bf16(src) element-wise, round to nearest even.
hipError_t launch_to_bf16(const float* src, bf16_t* dst, int64_t n, hipStream_t s);

hipError_t launch_combine(const void* y, bool y_bf16, const uint32_t* route_positions,
                          int64_t rows, int hidden, void* out, bool out_bf16, hipStream_t s);

// Weight packing helpers (registration time).
hipError_t launch_pack_w13_bf16(const void* const* w1, const void* const* w3, bool src_bf16,
                                bf16_t* dst, int experts, int ffn, int hidden, hipStream_t s);
hipError_t launch_pack_w2_bf16(const void* const* w2, bool src_bf16, bf16_t* dst, int experts, int ffn,
                               int hidden, hipStream_t s);

}  // namespace aps
