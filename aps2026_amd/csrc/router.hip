// Router: logits GEMM (bit-exact fp32 FMA chains) and quantised greedy top-2.
//
// Reference: k_matmul_transposed_narrow (src/tensor.cu:2943-3006) computes
// each logit as ONE fp32 accumulator walked over k = 0..H-1 with FMA, and
// k_moe_top2 (src/tensor.cu:1293-1331) quantises and greedy-selects.  The
// reference's own logs show that a last-ulp change upstream flips experts, so
// the chain order is fixed: no split-K, no tree reduction over k.
//
// gfx950 mapping.  The parallelism is T*E independent chains of length H.
// One lane owns one chain: a wavefront is 64 tokens x 1 expert, a workgroup
// 64 tokens x 4 experts (four waves sharing the x tile), grid [token tiles] x
// [E/4].  At T = 4096, E = 16 that is one wave per SIMD, so the time is the
// length of one dependent chain.  Measured on gfx950 (cycles per step):
// dependent v_fmac_f32_dpp alone 6.1; with the bf16 -> fp32 conversion
// interleaved 9.2; with the LDS operand reads 10.8; with the ring barrier
// 12.4.  The design keeps everything else off the chain:
//  * x streams into a two-slot LDS ring straight from global memory
//    (global_load_lds_dwordx4; no VGPR staging, no conversion pass).  A slot
//    holds 512 bytes of each of the 64 token rows, in 16-byte pieces XOR-
//    swizzled by row so that the 16 lanes of an LDS phase, each reading its
//    own row, hit 16 distinct 4-bank groups.  The copy of chunk c+1 is in
//    flight while chunk c (256 bf16 steps, ~1 us) is consumed.
//  * The gate chunk of the block's 4 experts rides in the same slot.  Lane
//    j of every 16-lane row reads gate value j of a 16-step group, and the
//    FMA takes it through DPP row_newbcast:j, which hands lane j's value to
//    the whole row: a broadcast that costs no LDS bandwidth and no scalar-
//    cache latency (scalar gate loads miss the scalar cache once per 64 B
//    and stall the chain on L2 latency).
//  * bf16 -> fp32 is exact (a shift or a mask).  The chain is one asm
//    stream in which the conversion for step j+2 sits behind the FMA of
//    step j; the FMA is v_fmac_f32_dpp(acc, gate_k, x_k), k ascending, as in
//    the reference (the product is commutative, so operand order does not
//    change a bit).
//  * Operand reads for block b+1 (32 steps) are issued before block b's
//    FMAs; the ring barrier for chunk c sits at the last block of chunk c-1,
//    so the first reads of a chunk are also issued ahead.
//  * 72 KB of LDS per workgroup: two workgroups per CU (two chains per SIMD
//    once T*E exceeds 64 chains per SIMD, T > 4096 at E = 16).
// With tiles % 8 == 0 the expert groups of a token tile land on one XCD
// (workgroups are dealt round-robin over the 8 XCDs), so x is fetched from
// HBM once per XCD L2.
#include "common.hpp"

namespace aps {
namespace {

constexpr int kRouterRowBytes = 512;        // bytes of one token row per chunk
constexpr int kRouterSlots = 2;             // LDS ring depth (chunks)
static_assert(kRouterSlots >= 2 && kRouterSlots <= 4, "chunk_ready() waits for at most two later chunks");
constexpr int kRouterPieces = kRouterRowBytes / 16;          // 16-byte pieces per row
constexpr int kRouterRowsPerCopy = kWave / kRouterPieces;    // rows per 1 KB copy
constexpr int kRouterXCopies = kRouterPieces / 4;            // x copies per wave per chunk
constexpr int kRouterExpertsPerBlock = 4;   // one wave per expert
constexpr int kRouterBlk = 32;              // chain steps per register block

typedef uint32_t ru32x4_t __attribute__((ext_vector_type(4)));

#define APS_RGP(p) ((const __attribute__((address_space(1))) void*)(p))
#define APS_RLP(p) ((__attribute__((address_space(3))) void*)(p))

template <bool XBF16>
struct RFmt {
    static constexpr int kElt = XBF16 ? 2 : 4;
    static constexpr int kK = kRouterRowBytes / kElt;                 // k per chunk (256 / 128)
    static constexpr int kBpc = kK / kRouterBlk;                      // blocks per chunk (8 / 4)
    static constexpr int kPieces = kRouterBlk * kElt / 16;            // 16-B x pieces per block (4 / 8)
    static constexpr int kXBytes = kWave * kRouterRowBytes;           // 32 KB
    static constexpr int kGBytes = kRouterExpertsPerBlock * kK * 4;   // 4 KB / 2 KB
    static constexpr int kSlotBytes = kXBytes + kGBytes;
    static constexpr int kGateDma = kK / kWave;                       // dword copies per wave (4 / 2)
    static constexpr int kDma = kRouterXCopies + kGateDma;            // copies per wave per chunk
};

// LDS byte offset of 16-byte piece c of token row r (0..63).
__device__ inline int rpos(int r, int c) { return r * kRouterRowBytes + ((c ^ (r & 15)) << 4); }

__device__ inline void r_wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (0x0 << 8) | (0x3 << 14)); }
template <int N>
__device__ inline void r_wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}
__device__ inline void r_barrier() { asm volatile("s_barrier" ::: "memory"); }

// ---- the chain: 32 steps per asm block --------------------------------------
// %0 acc; bf16: %1..%4 temporaries, %5 / %6 gate groups (steps 0-15 / 16-31),
// %7..%22 the 16 words of bf16 pairs.  Step 2i takes the low half of word i
// (shift), step 2i+1 the high half (mask).
#define APS_STR_(x) #x
#define APS_STR(x) APS_STR_(x)
#define APS_F(T, G, J) "v_fmac_f32_dpp %0, " G ", " T " row_newbcast:" APS_STR(J) " row_mask:0xf bank_mask:0xf\n\t"
#define APS_LO(T, W) "v_lshlrev_b32 " T ", 16, " W "\n\t"
#define APS_HI(T, W) "v_and_b32 " T ", 0xffff0000, " W "\n\t"
// Steps 4q .. 4q+3 (words W0 = 2q, in %1 / %2, and W1 = 2q+1) and the
// conversion of the next word WN into %1 / %2.
#define APS_QUAD(G, J, W1, WN)                                                          \
    APS_F("%1", G, J) APS_LO("%3", W1) APS_F("%2", G, J##_1) APS_HI("%4", W1)           \
    APS_F("%3", G, J##_2) APS_LO("%1", WN) APS_F("%4", G, J##_3) APS_HI("%2", WN)
#define APS_QUAD_LAST(G, J, W1)                                                         \
    APS_F("%1", G, J) APS_LO("%3", W1) APS_F("%2", G, J##_1) APS_HI("%4", W1)           \
    APS_F("%3", G, J##_2) APS_F("%4", G, J##_3)
// DPP lane numbers of the four steps of each quad
#define APS_J0 0
#define APS_J0_1 1
#define APS_J0_2 2
#define APS_J0_3 3
#define APS_J4 4
#define APS_J4_1 5
#define APS_J4_2 6
#define APS_J4_3 7
#define APS_J8 8
#define APS_J8_1 9
#define APS_J8_2 10
#define APS_J8_3 11
#define APS_J12 12
#define APS_J12_1 13
#define APS_J12_2 14
#define APS_J12_3 15

__device__ inline float chain32(float acc, float g0, float g1, const ru32x4_t (&xp)[4]) {
    float t0, t1, t2, t3;
    asm volatile(
        "s_nop 1\n\t"  // DPP source written by a VALU copy needs two wait states
        APS_LO("%1", "%7") APS_HI("%2", "%7")
        APS_QUAD("%5", APS_J0, "%8", "%9") APS_QUAD("%5", APS_J4, "%10", "%11")
        APS_QUAD("%5", APS_J8, "%12", "%13") APS_QUAD("%5", APS_J12, "%14", "%15")
        APS_QUAD("%6", APS_J0, "%16", "%17") APS_QUAD("%6", APS_J4, "%18", "%19")
        APS_QUAD("%6", APS_J8, "%20", "%21") APS_QUAD_LAST("%6", APS_J12, "%22")
        : "+v"(acc), "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3)
        : "v"(g0), "v"(g1),
          "v"(xp[0][0]), "v"(xp[0][1]), "v"(xp[0][2]), "v"(xp[0][3]),
          "v"(xp[1][0]), "v"(xp[1][1]), "v"(xp[1][2]), "v"(xp[1][3]),
          "v"(xp[2][0]), "v"(xp[2][1]), "v"(xp[2][2]), "v"(xp[2][3]),
          "v"(xp[3][0]), "v"(xp[3][1]), "v"(xp[3][2]), "v"(xp[3][3]));
    return acc;
}

// fp32 x: 16 steps, %0 acc, %1 gate group, %2..%17 the x values.
#define APS_F4(J, A, B, C, D) APS_F(A, "%1", J) APS_F(B, "%1", J##_1) APS_F(C, "%1", J##_2) APS_F(D, "%1", J##_3)
__device__ inline float chain16_f32(float acc, float g, const ru32x4_t& a, const ru32x4_t& b,
                                    const ru32x4_t& c, const ru32x4_t& d) {
    asm volatile(
        "s_nop 1\n\t"
        APS_F4(APS_J0, "%2", "%3", "%4", "%5") APS_F4(APS_J4, "%6", "%7", "%8", "%9")
        APS_F4(APS_J8, "%10", "%11", "%12", "%13") APS_F4(APS_J12, "%14", "%15", "%16", "%17")
        : "+v"(acc)
        : "v"(g), "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]),
          "v"(c[0]), "v"(c[1]), "v"(c[2]), "v"(c[3]), "v"(d[0]), "v"(d[1]), "v"(d[2]), "v"(d[3]));
    return acc;
}

template <bool XBF16>
__device__ inline float chain_block(float acc, float g0, float g1, const ru32x4_t (&xp)[RFmt<XBF16>::kPieces]) {
    if constexpr (XBF16) {
        return chain32(acc, g0, g1, xp);
    } else {
        acc = chain16_f32(acc, g0, xp[0], xp[1], xp[2], xp[3]);
        return chain16_f32(acc, g1, xp[4], xp[5], xp[6], xp[7]);
    }
}

template <bool XBF16>
__global__ void __launch_bounds__(256, 2)
k_router_logits(const void* __restrict__ xv, const float* __restrict__ gate, int64_t rows,
                int H, int E, float* __restrict__ logits) {
    using F = RFmt<XBF16>;
    // one LDS object: slot s = [x: 64 rows x 256 B][gate: 4 experts x kK floats]
    __shared__ __align__(16) uint8_t ring[kRouterSlots * F::kSlotBytes];

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int e = blockIdx.y * kRouterExpertsPerBlock + w;
    const bool active = e < E;  // wave-uniform
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kWave;
    const int NC = H / F::kK;   // chunks

    // x copies: copy j of a chunk fills x bytes [1024 j, 1024 j + 1024) = rows
    // R j .. R j + R - 1 (R = kRouterRowsPerCopy); wave w issues copies
    // X w .. X w + X - 1 (X = kRouterXCopies).  Lane i lands at piece
    // i % kRouterPieces of row R j + i / kRouterPieces and fetches the
    // logical piece that rpos() places there.  Rows past the end re-read the
    // last row.
    const uint8_t* xsrc[kRouterXCopies];
#pragma unroll
    for (int jj = 0; jj < kRouterXCopies; ++jj) {
        const int r = kRouterRowsPerCopy * (kRouterXCopies * w + jj) + lane / kRouterPieces;
        const int c = (lane % kRouterPieces) ^ (r & 15);
        const int64_t row = row0 + r < rows ? row0 + r : rows - 1;
        xsrc[jj] = static_cast<const uint8_t*>(xv) + row * static_cast<int64_t>(H) * F::kElt + c * 16;
    }
    // gate copies: wave w fetches expert e's kK values of the chunk, one
    // dword per lane per copy (inactive waves fetch a valid row, unused)
    const float* gsrc = gate + static_cast<int64_t>(active ? e : E - 1) * H + lane;
    auto issue_chunk = [&](int kc) {
        uint8_t* slot = ring + (kc % kRouterSlots) * F::kSlotBytes;
#pragma unroll
        for (int jj = 0; jj < kRouterXCopies; ++jj)
            __builtin_amdgcn_global_load_lds(APS_RGP(xsrc[jj] + static_cast<int64_t>(kc) * kRouterRowBytes),
                                             APS_RLP(slot + (kRouterXCopies * w + jj) * 1024), 16, 0, 0);
#pragma unroll
        for (int jj = 0; jj < F::kGateDma; ++jj)
            __builtin_amdgcn_global_load_lds(APS_RGP(gsrc + kc * F::kK + jj * kWave),
                                             APS_RLP(slot + F::kXBytes + w * F::kK * 4 + jj * 256), 4, 0, 0);
    };
    // chunk kc landed in this wave's view: wait for its copies (later chunks
    // may stay in flight), then the barrier makes every wave's copies visible
    auto chunk_ready = [&](int kc) {
        const int later = NC - 1 - kc < kRouterSlots - 2 ? NC - 1 - kc : kRouterSlots - 2;
        if (later >= 2) r_wait_vm<2 * F::kDma>();
        else if (later == 1) r_wait_vm<F::kDma>();
        else r_wait_vm<0>();
        r_barrier();
    };
    auto load_block = [&](ru32x4_t (&xp)[F::kPieces], float& g0, float& g1, int kc, int bb) {
        const uint8_t* slot = ring + (kc % kRouterSlots) * F::kSlotBytes;
#pragma unroll
        for (int p = 0; p < F::kPieces; ++p)
            xp[p] = *reinterpret_cast<const ru32x4_t*>(slot + rpos(lane, bb * F::kPieces + p));
        const float* gs = reinterpret_cast<const float*>(slot + F::kXBytes + w * F::kK * 4) + bb * kRouterBlk + (lane & 15);
        g0 = gs[0];
        g1 = gs[16];
    };

#pragma unroll
    for (int c = 0; c < kRouterSlots - 1; ++c)
        if (c < NC) issue_chunk(c);
    chunk_ready(0);
    if (kRouterSlots - 1 < NC) issue_chunk(kRouterSlots - 1);

    float acc = 0.0f;
    ru32x4_t xa[F::kPieces], xb[F::kPieces];
    float ga0, ga1, gb0, gb1;
    if (active) load_block(xa, ga0, ga1, 0, 0);
    for (int kc = 0; kc < NC; ++kc) {
        // register ping-pong: xa holds block bb, xb block bb + 1 (kBpc is even)
#pragma unroll
        for (int bb = 0; bb < F::kBpc; bb += 2) {
            if (active) {
                r_wait_lgkm0();
                load_block(xb, gb0, gb1, kc, bb + 1);
                __builtin_amdgcn_sched_barrier(0);
                acc = chain_block<XBF16>(acc, ga0, ga1, xa);
                __builtin_amdgcn_sched_barrier(0);
            }
            const bool last = bb + 2 == F::kBpc;
            if (last && kc + 1 < NC) {
                // chunk kc+1 opens next: this wave's reads of chunk kc are
                // done once block bb+1 has landed; after the barrier chunk
                // kc's slot is free for chunk kc + kRouterSlots
                if (active) r_wait_lgkm0();
                chunk_ready(kc + 1);
                if (kc + kRouterSlots < NC) issue_chunk(kc + kRouterSlots);
            }
            if (active) {
                r_wait_lgkm0();
                if (!last) load_block(xa, ga0, ga1, kc, bb + 2);
                else if (kc + 1 < NC) load_block(xa, ga0, ga1, kc + 1, 0);
                __builtin_amdgcn_sched_barrier(0);
                acc = chain_block<XBF16>(acc, gb0, gb1, xb);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    const int64_t row = row0 + lane;
    if (active && row < rows) logits[row * E + e] = acc;
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
        for (int e = 0; e < EMAX; ++e) q[e] = route_quantise(q[e]);
        route_greedy_top2<EMAX>(q, E, first, second);
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
    // whole chunks, and an even number of 32-step blocks
    if (hidden % (x_bf16 ? RFmt<true>::kK : RFmt<false>::kK) != 0 || experts <= 0) return hipErrorInvalidValue;
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
