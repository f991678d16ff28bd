// Router: logits GEMM (bit-exact fp32 FMA chains), quantised greedy top-2 and
// the per-tile expert histogram, in one kernel.
//
// Reference: k_matmul_transposed_narrow (src/tensor.cu:2943-3006) computes
// each logit as ONE fp32 accumulator walked over k = 0..H-1 with FMA, and
// k_moe_top2 (src/tensor.cu:1293-1331) quantises and greedy-selects.  A
// last-ulp change of a logit can flip an expert, so the chain order is fixed:
// no split-K, no tree reduction over k.
//
// gfx950 mapping.  There are T*E independent chains of length H and one lane
// owns one chain.  A wavefront is 4 tokens x 16 experts: each 16-lane row is
// one token and lane j of the row is expert j (E <= 16; for E <= 32 / 64 a
// token spans 2 / 4 rows, R = rows per token).  A workgroup is 16 tokens
// (4 R waves), so at T = 4096, E = 16 every SIMD runs one wave and the time
// is the length of one dependent chain.
//  * x is the broadcast operand.  Lane i of a row holds x[t][8i .. 8i+7] of a
//    128-step window (one 16-byte load per lane, straight to registers) and
//    v_fmac_f32_dpp ... row_newbcast:i hands element m of lane i to the whole
//    row.  The bf16 -> fp32 conversion (a shift or a mask, exact) costs 8
//    VALU ops per 128 steps instead of one per step.
//  * The gate is the per-lane operand.  128-step windows of every expert's
//    gate row sit in LDS as [k/4][expert][4] fp32, so the 16 lanes of a row
//    read 16 consecutive 16-byte pieces (no bank conflicts) and one
//    ds_read_b128 feeds four steps.  Windows stream into a two-stage LDS ring
//    with global_load_lds_dwordx4 (a stage is 32 KB: 512 steps of 16
//    experts), shared by the workgroup's waves, one barrier per stage.  Gate
//    reads run two 16-step blocks ahead of the FMAs.
//  * Each FMA is v_fmac_f32_dpp(acc, x_k, gate_k), k ascending, as in the
//    reference (the product is commutative, so the operand order changes no
//    bit).
//  * Measured on gfx950 (cycles per chain step, one wave per SIMD): the DPP
//    chain with its gate in registers 5.65, with the gate read from LDS 7.65.
//    A lane-per-token layout (x per lane from LDS and converted every step,
//    gate broadcast) ran at 12.4.
// After the chain a row holds its token's E logits.  Every lane gathers them
// (DPP row broadcasts), quantises and runs the reference's greedy scan; the
// workgroup's per-expert counts (one 16-token quarter of a 64-token tile)
// become one byte of the tile histogram words that the dispatch reads, and,
// when asked, the counts of slot-0 routes alone one byte of a second
// histogram (the dispatch's slot-ordered lists for the folded combine).
#include "common.hpp"

#include <utility>

namespace aps {
namespace {

constexpr int kRWin = 128;                // chain steps per window (one x load per lane)
constexpr int kRStageBytes = 32 * 1024;   // gate bytes per ring stage
constexpr int kRTokens = 16;              // tokens per workgroup: a quarter of a routing tile
static_assert(kTileTokens == 4 * kRTokens, "tile histogram words hold four quarter-tile bytes");

typedef uint32_t ru32x4_t __attribute__((ext_vector_type(4)));
typedef float rf32x4_t __attribute__((ext_vector_type(4)));

#define APS_RGP(p) ((const __attribute__((address_space(1))) void*)(p))
#define APS_RLP(p) ((__attribute__((address_space(3))) void*)(p))

template <int N>
__device__ inline void r_wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}
__device__ inline void r_wait_vm0() { r_wait_vm<0>(); }
__device__ inline void r_barrier() { asm volatile("s_barrier" ::: "memory"); }

// ---- the chain: 16 steps per asm block ---------------------------------------
// Step s = 0..15: acc = fma(x_s, g_s, acc), where x_s is element s % 8 of lane
// L0 (s < 8) or L1 (s >= 8) of the row, broadcast by DPP row_newbcast, and g_s
// this lane's gate value (g[s / 4][s % 4]).  Block b opens with the four gate
// reads of block b + 2 and then waits until 8 reads remain in flight: LDS
// reads complete in order, so that completes block b's own four (blocks b+1
// and b+2 stay in flight).  Measured on gfx950, the reads in one burst at the
// head of the block ran 7% faster than spread between the FMA groups.
// Operands: %0 acc; %1..%4 the next reads' destinations (early clobber: the
// data lands after the statement); %5..%12 x elements; %13..%28 gate values;
// %29 the lane's LDS address; %30..%33 the read offsets.
#define APS_RF(XI, GI, L) "v_fmac_f32_dpp %0, %" #XI ", %" #GI " row_newbcast:" #L " row_mask:0xf bank_mask:0xf\n\t"
#define APS_RG(L, X0, X1, X2, X3, G0, G1, G2, G3) APS_RF(X0, G0, L) APS_RF(X1, G1, L) APS_RF(X2, G2, L) APS_RF(X3, G3, L)
#define APS_RBODY(L0, L1)                        \
    APS_RG(L0, 5, 6, 7, 8, 13, 14, 15, 16)       \
    APS_RG(L0, 9, 10, 11, 12, 17, 18, 19, 20)    \
    APS_RG(L1, 5, 6, 7, 8, 21, 22, 23, 24)       \
    APS_RG(L1, 9, 10, 11, 12, 25, 26, 27, 28)
#define APS_RREADS                                 \
    "ds_read_b128 %1, %29 offset:%30\n\t"          \
    "ds_read_b128 %2, %29 offset:%31\n\t"          \
    "ds_read_b128 %3, %29 offset:%32\n\t"          \
    "ds_read_b128 %4, %29 offset:%33\n\t"
#define APS_RBLK(NAME, HEAD, L0, L1)                                                                      \
    template <int OFF, int STRIDE>                                                                        \
    __device__ inline float NAME(float acc, const float (&c)[8], const rf32x4_t (&g)[4], rf32x4_t (&gn)[4], \
                                 uint32_t addr) {                                                         \
        asm volatile(HEAD APS_RBODY(L0, L1)                                                               \
                     : "+v"(acc), "=&v"(gn[0]), "=&v"(gn[1]), "=&v"(gn[2]), "=&v"(gn[3])                  \
                     : "v"(c[0]), "v"(c[1]), "v"(c[2]), "v"(c[3]), "v"(c[4]), "v"(c[5]), "v"(c[6]),       \
                       "v"(c[7]), "v"(g[0][0]), "v"(g[0][1]), "v"(g[0][2]), "v"(g[0][3]), "v"(g[1][0]),   \
                       "v"(g[1][1]), "v"(g[1][2]), "v"(g[1][3]), "v"(g[2][0]), "v"(g[2][1]), "v"(g[2][2]), \
                       "v"(g[2][3]), "v"(g[3][0]), "v"(g[3][1]), "v"(g[3][2]), "v"(g[3][3]), "v"(addr),   \
                       "n"(OFF), "n"(OFF + STRIDE), "n"(OFF + 2 * STRIDE), "n"(OFF + 3 * STRIDE));         \
        return acc;                                                                                       \
    }
// Block 0 of a window follows the VALU writes of its x elements: a DPP
// source written by VALU needs two wait states (the reads provide them).
APS_RBLK(rblk0, APS_RREADS "s_waitcnt lgkmcnt(8)\n\t", 0, 1)
APS_RBLK(rblk1, APS_RREADS "s_waitcnt lgkmcnt(8)\n\t", 2, 3)
APS_RBLK(rblk2, APS_RREADS "s_waitcnt lgkmcnt(8)\n\t", 4, 5)
APS_RBLK(rblk3, APS_RREADS "s_waitcnt lgkmcnt(8)\n\t", 6, 7)
APS_RBLK(rblk4, APS_RREADS "s_waitcnt lgkmcnt(8)\n\t", 8, 9)
APS_RBLK(rblk5, APS_RREADS "s_waitcnt lgkmcnt(8)\n\t", 10, 11)
APS_RBLK(rblk6, APS_RREADS "s_waitcnt lgkmcnt(8)\n\t", 12, 13)
APS_RBLK(rblk7, APS_RREADS "s_waitcnt lgkmcnt(8)\n\t", 14, 15)
// the last two blocks of a stage read nothing ahead
APS_RBLK(rblk6_tail, "s_waitcnt lgkmcnt(4)\n\t", 12, 13)
APS_RBLK(rblk7_tail, "s_waitcnt lgkmcnt(0)\n\t", 14, 15)

// Block b of a stage of NB blocks (NB a multiple of 8): the FMAs of block b,
// with the reads of block b + 2 (offsets OFF + m STRIDE) when it exists.
template <int B, int NB, int OFF, int STRIDE>
__device__ inline float rblock(float acc, const float (&c)[8], const rf32x4_t (&g)[4], rf32x4_t (&gn)[4],
                               uint32_t addr) {
    constexpr int Q = B % 8;
    if constexpr (B == NB - 2) return rblk6_tail<0, 0>(acc, c, g, gn, addr);
    else if constexpr (B == NB - 1) return rblk7_tail<0, 0>(acc, c, g, gn, addr);
    else if constexpr (Q == 0) return rblk0<OFF, STRIDE>(acc, c, g, gn, addr);
    else if constexpr (Q == 1) return rblk1<OFF, STRIDE>(acc, c, g, gn, addr);
    else if constexpr (Q == 2) return rblk2<OFF, STRIDE>(acc, c, g, gn, addr);
    else if constexpr (Q == 3) return rblk3<OFF, STRIDE>(acc, c, g, gn, addr);
    else if constexpr (Q == 4) return rblk4<OFF, STRIDE>(acc, c, g, gn, addr);
    else if constexpr (Q == 5) return rblk5<OFF, STRIDE>(acc, c, g, gn, addr);
    else if constexpr (Q == 6) return rblk6<OFF, STRIDE>(acc, c, g, gn, addr);
    else return rblk7<OFF, STRIDE>(acc, c, g, gn, addr);
}

// x elements of one window as fp32, produced by asm so that the compiler can
// neither recompute nor copy them next to a DPP read.  bf16: element 2p is
// the low half of word p (shift), 2p+1 the high half (mask); both exact.
__device__ inline void r_elements(float (&c)[8], const ru32x4_t (&w)[1]) {
    asm volatile(
        "v_lshlrev_b32 %0, 16, %8\n\t"
        "v_and_b32 %1, 0xffff0000, %8\n\t"
        "v_lshlrev_b32 %2, 16, %9\n\t"
        "v_and_b32 %3, 0xffff0000, %9\n\t"
        "v_lshlrev_b32 %4, 16, %10\n\t"
        "v_and_b32 %5, 0xffff0000, %10\n\t"
        "v_lshlrev_b32 %6, 16, %11\n\t"
        "v_and_b32 %7, 0xffff0000, %11\n\t"
        : "=&v"(c[0]), "=&v"(c[1]), "=&v"(c[2]), "=&v"(c[3]), "=&v"(c[4]), "=&v"(c[5]), "=&v"(c[6]), "=&v"(c[7])
        : "v"(w[0][0]), "v"(w[0][1]), "v"(w[0][2]), "v"(w[0][3]));
}
__device__ inline void r_elements(float (&c)[8], const ru32x4_t (&w)[2]) {
    asm volatile(
        "v_mov_b32 %0, %8\n\t"
        "v_mov_b32 %1, %9\n\t"
        "v_mov_b32 %2, %10\n\t"
        "v_mov_b32 %3, %11\n\t"
        "v_mov_b32 %4, %12\n\t"
        "v_mov_b32 %5, %13\n\t"
        "v_mov_b32 %6, %14\n\t"
        "v_mov_b32 %7, %15\n\t"
        : "=&v"(c[0]), "=&v"(c[1]), "=&v"(c[2]), "=&v"(c[3]), "=&v"(c[4]), "=&v"(c[5]), "=&v"(c[6]), "=&v"(c[7])
        : "v"(w[0][0]), "v"(w[0][1]), "v"(w[0][2]), "v"(w[0][3]), "v"(w[1][0]), "v"(w[1][1]), "v"(w[1][2]),
          "v"(w[1][3]));
}

// The four gate reads of one 16-step block (byte offsets OFF + m STRIDE from
// the lane's LDS address), for the first two blocks of a stage.  Reads are
// issued from asm and waited for inside the chain blocks: the compiler would
// drain them before every block; the outputs are early-clobber since the data
// lands after the statement.
template <int OFF, int STRIDE>
__device__ inline void r_gate_reads(rf32x4_t (&gd)[4], uint32_t addr) {
    asm volatile(
        "ds_read_b128 %0, %4 offset:%5\n\t"
        "ds_read_b128 %1, %4 offset:%6\n\t"
        "ds_read_b128 %2, %4 offset:%7\n\t"
        "ds_read_b128 %3, %4 offset:%8"
        : "=&v"(gd[0]), "=&v"(gd[1]), "=&v"(gd[2]), "=&v"(gd[3])
        : "v"(addr), "n"(OFF), "n"(OFF + STRIDE), "n"(OFF + 2 * STRIDE), "n"(OFF + 3 * STRIDE));
}
template <int V>
struct RInt {
    static constexpr int value = V;
    constexpr operator int() const { return V; }
};

// Two fp32 -> packed bf16, round to nearest even (v_cvt_pk_bf16_f32), the
// same conversion as the library's standalone fp32 -> bf16 kernel.
__device__ inline uint32_t r_pack2_bf16(float lo, float hi) {
    typedef __bf16 rbf16x2_t __attribute__((ext_vector_type(2)));
    rbf16x2_t v;
    v[0] = static_cast<__bf16>(lo);
    v[1] = static_cast<__bf16>(hi);
    return __builtin_bit_cast(uint32_t, v);
}

// One workgroup = 16 tokens x 16 R expert lanes.  logits [rows][E] always;
// routes [rows][2] and the tile histogram when routes != nullptr.  XCOPY
// (fp32 x only): the bf16 copy of x the expert FFN reads is written on the
// way, each lane storing its 8 converted elements of every window (the R
// rows of a token and the clamped rows past the end store identical values),
// which spares the FFN path a separate conversion pass over x.  A ring
// stage holds GW windows; H is a multiple of GW * 128, so every stage is full
// and the step sequence has no run-time bounds (the compiler can then count
// the LDS reads in flight instead of draining them).
// NWV waves per 16 R lanes of experts: 4 (16 tokens per workgroup) or, for
// R = 1 and large batches, 8 (32 tokens): the gate then streams once per 32
// tokens instead of once per 16, half the gate copies per CU.
// XQS > 0 (bf16 x, R = 1, H = XQS stages): the fp8 path's x quantisation on
// the way.  Each lane keeps the raw x words it loads for the chain (XQS * GW
// windows of 8 bf16 values: 4 XQS GW registers), and after the chain its row
// reduces the token's amax over its 16 lanes and every lane writes the e4m3
// codes of its own elements and lane 0 the row's scale, with the row
// quantiser's arithmetic (common.hpp), so the codes and scales are the ones
// k_quant_rows writes.  x is read from memory once for both.
template <bool XBF16, int R, int GW, bool XCOPY = false, int NWV = 4, int XQS = 0>
__global__ void __launch_bounds__(64 * NWV * R)
k_router(const void* xv, const float* __restrict__ gate, int64_t rows, int H, int E,
         float* __restrict__ logits, uint8_t* __restrict__ routes, uint8_t* __restrict__ tile_bytes,
         uint8_t* __restrict__ tile_bytes0, bf16_t* __restrict__ xcopy, uint8_t* __restrict__ xq,
         float* __restrict__ xq_scale) {
    static_assert(!(XCOPY && XBF16), "the bf16 copy is made from fp32 x");
    static_assert(XQS == 0 || (XBF16 && R == 1 && !XCOPY), "x quantisation reads bf16 x, one row per token");
    constexpr int kGW = GW;                    // windows per ring stage
    constexpr int kWinBytes = 8 * 1024 * R;    // 32 (k/4) x 16 R experts x 16 B
    constexpr int kElt = XBF16 ? 2 : 4;
    constexpr int kXv = XBF16 ? 1 : 2;         // 16-byte x loads per lane per window
    constexpr int kStageBytes = kGW * kWinBytes;
    static_assert(kStageBytes <= kRStageBytes, "stage geometry");
    // two LDS objects, so that the compiler sees the stage being filled and
    // the stage being read as distinct memory
    __shared__ __align__(16) uint8_t ring0[kStageBytes];
    __shared__ __align__(16) uint8_t ring1[kStageBytes];
    constexpr int kWaves = NWV * R;            // waves per workgroup
    constexpr int kTok = 4 * NWV;              // tokens per workgroup
    constexpr int kQ = kTok / kRTokens;        // routing-tile quarters per workgroup
    static_assert(R == 1 || NWV == 4, "eight-wave workgroups for E <= 16");
    // [0]: the quarters' route counts per expert, [1]: slot-0 routes only
    // (tile_bytes0)
    __shared__ uint32_t cnt[2][kQ][16 * R];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gr = 4 * w + (lane >> 4);        // row of the workgroup, 0 .. 16R-1
    const int e = (gr % R) * 16 + (lane & 15); // this lane's expert
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kTok + gr / R;
    // stages: compile-time when the x words are kept (their registers are
    // indexed by stage), H = XQS GW 128 then
    const int NG = XQS > 0 ? XQS : H / kRWin / kGW;
    static_assert(2 * kQ * 16 * R <= 64 * NWV * R, "one counter per thread to clear");
    if (tid < 2 * kQ * 16 * R) (&cnt[0][0][0])[tid] = 0u;

    // x: lane i of a row reads elements 8i .. 8i+7 of every window of its
    // token (rows past the end re-read the last row; their results are
    // dropped)
    const uint8_t* xsrc = static_cast<const uint8_t*>(xv) +
                          ((t < rows ? t : rows - 1) * static_cast<int64_t>(H) + 8 * (lane & 15)) * kElt;
    bf16_t* xdst = XCOPY ? xcopy + (t < rows ? t : rows - 1) * static_cast<int64_t>(H) + 8 * (lane & 15) : nullptr;
    // gate copies: a window is 8 R copies of 1 KB; copy i of a stage
    // (i = 0 .. 8 R kGW / kWaves - 1) is instruction a = w + kWaves i of the
    // stage and fills bytes [a KB, a KB + 1 KB): window a / 8R of the stage,
    // piece (a % 8R) * 64 + lane of the window, i.e. k/4 = piece / 16R and
    // expert piece % 16R.  Padding experts read row E-1 (unused).
    constexpr int kPieces = 8 * R / kWaves > 0 ? 8 * R / kWaves : 1;   // distinct pieces per lane
    constexpr int kCopies = 8 * R * kGW / kWaves;                     // copies per wave per stage
    const float* gsrc[kPieces];
#pragma unroll
    for (int p = 0; p < kPieces; ++p) {
        const int piece = (w + kWaves * p) * 64 + lane;
        const int ge = piece % (16 * R);
        gsrc[p] = gate + static_cast<int64_t>(ge < E ? ge : E - 1) * H + 4 * (piece / (16 * R));
    }
    auto issue_gate = [&](auto par, int g) {
        uint8_t* slot = decltype(par)::value ? ring1 : ring0;
        const int v0 = g * kGW;
#pragma unroll
        for (int i = 0; i < kCopies; ++i)
            __builtin_amdgcn_global_load_lds(APS_RGP(gsrc[i % kPieces] + (v0 + i / kPieces) * kRWin),
                                             APS_RLP(slot + (w + kWaves * i) * 1024), 16, 0, 0);
    };
    ru32x4_t xr[2][kGW][kXv];
    auto issue_x = [&](ru32x4_t (&dst)[kGW][kXv], int g) {
        const int v0 = g * kGW;
#pragma unroll
        for (int wi = 0; wi < kGW; ++wi)
#pragma unroll
            for (int p = 0; p < kXv; ++p)
                dst[wi][p] = *reinterpret_cast<const ru32x4_t*>(xsrc + (v0 + wi) * kRWin * kElt + p * 16);
    };
    // gate values of block b (window b / 8, steps 16 (b % 8) .. +15) of a
    // stage: piece (4 (b % 8) + m) * 16R + e of window b / 8, i.e. byte
    // gate_off(b) + m * kGateStride from the lane's address
    const uint32_t gaddr0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(APS_RLP(ring0))) + e * 16;
    const uint32_t gaddr1 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(APS_RLP(ring1))) + e * 16;
    constexpr int kGateStride = 16 * R * 16;  // bytes per k/4 row of a window
    constexpr auto gate_off = [](int b) constexpr { return (b / 8) * kWinBytes + 4 * (b % 8) * kGateStride; };
    auto load_gate = [&](rf32x4_t (&gd)[4], uint32_t addr, auto bq) {
        constexpr int b = decltype(bq)::value;
        r_gate_reads<gate_off(b), kGateStride>(gd, addr);
    };

    // the raw x words of every window, for the quantisation after the chain
    ru32x4_t xs[XQS > 0 ? XQS * kGW : 1];

    float acc = 0.0f;
    // stage g (an int, or an RInt when the x words are kept)
    auto run_stage = [&](auto par, auto gq) {
        constexpr int P = decltype(par)::value;
        const int g = gq;
        constexpr int nb = 8 * kGW;
        // this stage's x elements, then the next stage's x loads (the x
        // registers of this stage are free once converted)
        float c[kGW][8];
#pragma unroll
        for (int wi = 0; wi < kGW; ++wi) r_elements(c[wi], xr[P][wi]);
        if constexpr (XQS > 0) {
            constexpr int G = decltype(gq)::value;
#pragma unroll
            for (int wi = 0; wi < kGW; ++wi) xs[G * kGW + wi] = xr[P][wi][0];
        }
        if constexpr (XCOPY) {
#pragma unroll
            for (int wi = 0; wi < kGW; ++wi) {
                const ru32x4_t pk = {r_pack2_bf16(c[wi][0], c[wi][1]), r_pack2_bf16(c[wi][2], c[wi][3]),
                                     r_pack2_bf16(c[wi][4], c[wi][5]), r_pack2_bf16(c[wi][6], c[wi][7])};
                *reinterpret_cast<ru32x4_t*>(xdst + (g * kGW + wi) * kRWin) = pk;
            }
        }
        if (g + 1 < NG) issue_x(xr[P ^ 1], g + 1);
        const uint32_t gaddr = P ? gaddr1 : gaddr0;
        rf32x4_t gs[3][4];
        load_gate(gs[0], gaddr, RInt<0>{});
        load_gate(gs[1], gaddr, RInt<1>{});
        rf32x4_t spare[4];  // destinations of the last two blocks' (absent) reads
        auto step = [&](auto bq) {
            constexpr int b = decltype(bq)::value;
            if constexpr (b + 2 < nb)
                acc = rblock<b, nb, gate_off(b + 2), kGateStride>(acc, c[b / 8], gs[b % 3], gs[(b + 2) % 3], gaddr);
            else
                acc = rblock<b, nb, 0, kGateStride>(acc, c[b / 8], gs[b % 3], spare, gaddr);
        };
        [&]<int... B>(std::integer_sequence<int, B...>) { (step(RInt<B>{}), ...); }(
            std::make_integer_sequence<int, 8 * kGW>{});
        // the next stage's gate and x have landed (every copy, in order);
        // after the barrier all waves see the gate and this stage's slot is
        // free for stage g + 2.  Unconditional, so that on every path the x
        // registers are complete before their next use.
        r_wait_vm0();
        r_barrier();
        if (g + 2 < NG) issue_gate(par, g + 2);
    };

    // stage 0 needs its gate and x; stage 1's gate copies (the last kCopies
    // per wave) may stay in flight.  With a single stage the second slot is
    // filled with stage 0 again (unused), so the wait is the same on every
    // path and the compiler sees the x registers complete.
    issue_gate(RInt<0>{}, 0);
    issue_x(xr[0], 0);
    issue_gate(RInt<1>{}, NG > 1 ? 1 : 0);
    r_wait_vm<kCopies>();
    r_barrier();
    if constexpr (XQS > 0) {
        [&]<int... G>(std::integer_sequence<int, G...>) { (run_stage(RInt<G % 2>{}, RInt<G>{}), ...); }(
            std::make_integer_sequence<int, XQS>{});
    } else {
        for (int g = 0; g < NG; g += 2) {
            run_stage(RInt<0>{}, g);
            if (g + 1 < NG) run_stage(RInt<1>{}, g + 1);
        }
    }

    const bool valid = t < rows;
    if (valid && e < E) logits[t * E + e] = acc;
    if constexpr (XQS > 0) {
        // the token's row scale (its 16 lanes hold the whole row), then the
        // codes of this lane's 8 elements of every window
        float amax = 0.0f;
#pragma unroll
        for (int v = 0; v < XQS * kGW; ++v) amax = e4m3_amax8(amax, xs[v]);
#pragma unroll
        for (int d = 8; d >= 1; d >>= 1) amax = fmaxf(amax, __shfl_xor(amax, d));
        const float sc = e4m3_row_scale(amax);
        const float rc = __fdiv_rn(1.0f, sc);
        if (valid) {
            if ((lane & 15) == 0) xq_scale[t] = sc;
            typedef uint32_t ru32x2_t __attribute__((ext_vector_type(2)));
            uint8_t* d8 = xq + t * static_cast<int64_t>(H) + 8 * (lane & 15);
            // The words pass through an empty asm statement, so that the
            // compiler converts them again here instead of keeping all 256
            // fp32 values of the amax loop alive (which spilled).
            if (sc >= kMinFastScale) {
#pragma unroll
                for (int v = 0; v < XQS * kGW; ++v) {
                    e4m3_words_t wv = xs[v];
                    asm volatile("" : "+v"(wv));
                    uint32_t lo, hi;
                    e4m3_chunk_codes<true>(wv, sc, rc, lo, hi);
                    *reinterpret_cast<ru32x2_t*>(d8 + v * kRWin) = ru32x2_t{lo, hi};
                }
            } else {
#pragma unroll
                for (int v = 0; v < XQS * kGW; ++v) {
                    e4m3_words_t wv = xs[v];
                    asm volatile("" : "+v"(wv));
                    uint32_t lo, hi;
                    e4m3_chunk_codes<false>(wv, sc, rc, lo, hi);
                    *reinterpret_cast<ru32x2_t*>(d8 + v * kRWin) = ru32x2_t{lo, hi};
                }
            }
        }
    }
    if (routes == nullptr) return;  // kernel-uniform

    // top-2 of the token: its 16 R logits sit in lanes base .. base + 16R - 1
    const float q = route_quantise(acc);
    const int base = lane & ~(16 * R - 1);
    float qs[16 * R];
    if constexpr (R == 1) {
        // the token's 16 values sit in its 16-lane row: DPP row broadcasts
        const int qi = __builtin_bit_cast(int, q);
        [&]<int... K>(std::integer_sequence<int, K...>) __attribute__((always_inline)) {
            ((qs[K] = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(qi, 0x150 + K, 0xF, 0xF, false))), ...);
        }(std::make_integer_sequence<int, 16>{});
    } else {
#pragma unroll
        for (int k = 0; k < 16 * R; ++k) qs[k] = __shfl(q, base + k);
    }
    int first, second;
    route_greedy_top2<16 * R>(qs, E, first, second);
    if (valid && lane == base) {
        routes[2 * t] = static_cast<uint8_t>(first);
        routes[2 * t + 1] = static_cast<uint8_t>(second);
    }
    if (valid && e < E && (e == first || e == second)) atomicAdd(&cnt[0][(gr / R) / kRTokens][e], 1u);
    if (tile_bytes0 && valid && e < E && e == first) atomicAdd(&cnt[1][(gr / R) / kRTokens][e], 1u);
    __syncthreads();
    if (tid < kQ * E) {
        // byte (quarter % 4) of word [tile][expert]; the last workgroup also
        // zeroes the bytes of quarters past the end
        const int qi = tid / E, ex = tid % E;
        const int64_t quarter = static_cast<int64_t>(blockIdx.x) * kQ + qi;
        const int sub = static_cast<int>(quarter % 4);
        uint8_t* word = tile_bytes + ((quarter / 4) * E + ex) * 4;
        word[sub] = static_cast<uint8_t>(cnt[0][qi][ex]);
        if (blockIdx.x == gridDim.x - 1 && qi == kQ - 1)
            for (int s2 = sub + 1; s2 < 4; ++s2) word[s2] = 0;
        if (tile_bytes0) {
            uint8_t* word0 = tile_bytes0 + ((quarter / 4) * E + ex) * 4;
            word0[sub] = static_cast<uint8_t>(cnt[1][qi][ex]);
            if (blockIdx.x == gridDim.x - 1 && qi == kQ - 1)
                for (int s2 = sub + 1; s2 < 4; ++s2) word0[s2] = 0;
        }
    }
}

// Top-2 from logits given by the caller (the reference's k_moe_top2 stage):
// one thread per token, one 64-thread workgroup per 64-token tile.  The
// token's E logits are loaded up front (independent loads, one round trip),
// then quantised and scanned twice.  Writes routes and, when asked, the
// tile's histogram words (popcounts of wave ballots: no atomics).
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
            const uint32_t c = tile_quarter_counts(first, second, e);
            if (lane == e) mine = c;
        }
        if (lane < E) tile_counts[tile * E + lane] = mine;
    }
}

}  // namespace

// Stages of 512 steps the router's x quantisation keeps in registers.
constexpr int kXqStages = 8;

bool router_quantises_x(int hidden, int experts) {
    return experts >= 1 && experts <= 16 && hidden == kXqStages * 4 * kRWin;
}

hipError_t launch_router(const void* x, bool x_bf16, const float* gate, int64_t rows, int hidden,
                         int experts, float* logits, uint8_t* routes, uint32_t* tile_counts,
                         uint32_t* tile_counts0, bf16_t* x_copy, uint8_t* xq, float* xq_scale, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hidden <= 0 || hidden % (2 * kRWin) != 0 || experts <= 0 || experts > kMaxExperts)
        return hipErrorInvalidValue;
    if (routes && (experts < 2 || !tile_counts)) return hipErrorInvalidValue;
    if (tile_counts0 && !routes) return hipErrorInvalidValue;
    if (x_copy && x_bf16) return hipErrorInvalidValue;
    if ((xq != nullptr) != (xq_scale != nullptr)) return hipErrorInvalidValue;
    if (xq && (!x_bf16 || !router_quantises_x(hidden, experts))) return hipErrorInvalidValue;
    auto* tb = reinterpret_cast<uint8_t*>(tile_counts);
    auto* tb0 = reinterpret_cast<uint8_t*>(tile_counts0);
    // windows per stage: 512 steps of 16 R experts (32 KB) when H allows
    const int R = experts <= 16 ? 1 : experts <= 32 ? 2 : 4;
    const bool wide = hidden % (4 * kRWin) == 0;
    // 32-token workgroups when 16-token ones would put two on some CU and
    // 32-token ones at most one on each (C5's 8,192 tokens): the CU then
    // streams the gate once for its 32 tokens.  Past that (C4's 10,240 rows)
    // some CUs would hold two 32-token workgroups, which measured slower.
    const int64_t cus = num_cus();
    const bool eight = R == 1 && wide && rows > kRTokens * cus && ceil_div(rows, 2 * kRTokens) <= cus;
    const dim3 grid(static_cast<unsigned>(ceil_div(rows, eight ? 2 * kRTokens : kRTokens)));
    if (xq) {
        if (eight)
            hipLaunchKernelGGL((k_router<true, 1, 4, false, 8, kXqStages>), grid, dim3(64 * 8), 0, s, x, gate, rows,
                               hidden, experts, logits, routes, tb, tb0, nullptr, xq, xq_scale);
        else
            hipLaunchKernelGGL((k_router<true, 1, 4, false, 4, kXqStages>), grid, dim3(64 * 4), 0, s, x, gate, rows,
                               hidden, experts, logits, routes, tb, tb0, nullptr, xq, xq_scale);
        return hipGetLastError();
    }
#define APS_ROUTER_LAUNCH(XB, R, GW, NWV)                                                                     \
    do {                                                                                                      \
        if (!(XB) && x_copy)                                                                                 \
            hipLaunchKernelGGL((k_router<false, R, GW, true, NWV>), grid, dim3(64 * NWV * R), 0, s, x, gate, \
                               rows, hidden, experts, logits, routes, tb, tb0, x_copy, nullptr, nullptr);    \
        else                                                                                                 \
            hipLaunchKernelGGL((k_router<XB, R, GW, false, NWV>), grid, dim3(64 * NWV * R), 0, s, x, gate,   \
                               rows, hidden, experts, logits, routes, tb, tb0, nullptr, nullptr, nullptr);   \
    } while (0)
    if (x_bf16) {
        if (eight) APS_ROUTER_LAUNCH(true, 1, 4, 8);
        else if (R == 1 && wide) APS_ROUTER_LAUNCH(true, 1, 4, 4);
        else if (R == 1) APS_ROUTER_LAUNCH(true, 1, 2, 4);
        else if (R == 2) APS_ROUTER_LAUNCH(true, 2, 2, 4);
        else APS_ROUTER_LAUNCH(true, 4, 1, 4);
    } else {
        if (eight) APS_ROUTER_LAUNCH(false, 1, 4, 8);
        else if (R == 1 && wide) APS_ROUTER_LAUNCH(false, 1, 4, 4);
        else if (R == 1) APS_ROUTER_LAUNCH(false, 1, 2, 4);
        else if (R == 2) APS_ROUTER_LAUNCH(false, 2, 2, 4);
        else APS_ROUTER_LAUNCH(false, 4, 1, 4);
    }
#undef APS_ROUTER_LAUNCH
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
