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
//  * w1/w3 and w2 are re-packed at registration into swizzled 128 x 64 tile
//    images (launch_pack_*): each B stage is one contiguous 16 KB block whose
//    bytes are copied to LDS unchanged.
//  * The token gather of the w1||w3 kernel is an index on the A load, as in
//    the reference: no permuted copy of x is ever written.
//  * Work list: (row tile, column block) pairs over all experts (sum_e
//    ceil(count_e / 128) row tiles), dealt to XCDs in contiguous slices so
//    operand reuse stays inside one L2; each block finds its expert from
//    offsets[] with a wave-uniform scan (scalar loads), so skewed experts
//    simply own more tiles and no host round trip is needed.
#include <cstdlib>

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

// Element offset of 16-byte chunk `chunk` (0..7) of tile row `row`.  gfx950's
// LDS has 64 four-byte banks (a 256-byte bank row = two 128-byte tile rows)
// and serves a ds_read_b128 16 lanes at a time.  An MFMA operand fetch reads
// the same logical chunk from 16 consecutive rows, so the physical chunk is
// chunk ^ ((row >> 1) & 7): rows 2m and 2m+1 sit in the two halves of a bank
// row, and the eight pairs of a 16-row group get eight different chunks --
// sixteen distinct 16-byte bank groups, no conflict.
__device__ inline int swz(int row, int chunk) { return row * kBK + ((chunk ^ ((row >> 1) & 7)) << 3); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ inline bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ inline f32x16_t mfma(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// XCD-aware tile map.  The work is a list of (row tile, column block)
// pairs, row-tile major: row tiles run over experts in order, each expert
// owning ceil(count_e / bm) of them.  Workgroups are dealt round-robin to the
// 8 XCDs (workgroup b runs on XCD b % 8), so XCD x takes the contiguous slice
// [x * per, (x + 1) * per) of the list: the column blocks of one row tile
// (sharing A rows) and the row tiles of one expert (sharing B) then meet in
// one XCD's L2 instead of being fetched by all eight.  Returns false for
// workgroups past the end of the list (the grid is sized for the worst case).
constexpr int kXcds = 8;

__device__ inline bool locate_tile(const uint32_t* __restrict__ offsets, int E, int bm, int n_blocks,
                                   int& expert, uint32_t& m0, uint32_t& end, int& nb) {
    uint32_t lo, hi;
    int incl;
    const int total_m = wave_tile_scan(offsets, E, bm, lo, hi, incl);
    const int total = total_m * n_blocks;
    const int b = blockIdx.x;
    const int per = (total + kXcds - 1) / kXcds;
    const int l = b / kXcds;
    const int t = (b % kXcds) * per + l;
    if (l >= per || t >= total) return false;
    const int tile = t / n_blocks;
    nb = t - tile * n_blocks;
    const RowTile r = wave_find_tile(tile, bm, lo, hi, incl, E);
    expert = r.expert;
    m0 = r.m0;
    end = r.end;
    return true;
}

// The 32x32 MFMA accumulator layout: register v of lane l holds
// D[8 * (v / 4) + 4 * (l / 32) + v % 4][l % 32].  With the B operand first
// (see mma()), D's row index is the output column: register group q = v / 4
// of lane l covers output columns 8q + 4 * (l / 32) .. +3 of token row l % 32.

// Two fp32 -> packed bf16, round to nearest even (one v_cvt_pk_bf16_f32).
__device__ inline uint32_t pack2_bf16(float lo, float hi) {
    bf16x2_t v;
    v[0] = static_cast<__bf16>(lo);
    v[1] = static_cast<__bf16>(hi);
    return __builtin_bit_cast(uint32_t, v);
}

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// silu(g) * u for the bf16 path: fp32 math with the hardware exp2 and
// reciprocal (result is rounded to bf16, far coarser than their error).
__device__ inline float swiglu(float g, float u) {
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

// ---------------------------------------------------------------------------
// Shared main loop.  A and B tiles (128 rows x 64 k each) stream from global
// memory straight into an S-stage LDS ring with global_load_lds_dwordx4 (no
// VGPR staging): lane i of a wave writes LDS bytes [16i, 16i+16) of a 1 KB
// slot = 8 tile rows, so the XOR swizzle is applied on the global side: lane
// i fetches the logical chunk that swz() places at its slot.
// Each wave issues 4 A + 4 B loads per stage (rows 32w .. 32w+31).  With the
// swizzle of swz(), lane i of load j (rows 32w + 8j + i/8) fetches logical
// chunk (i & 7) ^ ((4 * (j & 1) + (i >> 4)) & 7).  Loads
// run S-1 stages ahead; before consuming stage kt a wave waits until at most
// the loads of the later stages are outstanding (vmcnt), then one s_barrier
// publishes the stage to all waves and retires the oldest slot for reuse.
// The barrier is a raw s_barrier (not __syncthreads, whose workgroup fence
// would drain every in-flight load and serialise the ring).

struct RowPtrs {
    const bf16_t* p0;
    const bf16_t* p1;
    const bf16_t* p2;
    const bf16_t* p3;
};

#define APS_GP(p) ((const __attribute__((address_space(1))) void*)(p))
#define APS_LP(p) ((__attribute__((address_space(3))) void*)(p))

__device__ inline void dma16(const bf16_t* src, bf16_t* lds_slot) {
    __builtin_amdgcn_global_load_lds(APS_GP(src), APS_LP(lds_slot), 16, 0, 0);
}

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] |
// lgkmcnt[11:8] | vmcnt[5:4] at bits [15:14]); n must be a constant.
template <int N>
__device__ inline void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
}

__device__ inline void raw_barrier() { asm volatile("s_barrier" ::: "memory"); }

// s_waitcnt lgkmcnt(0) alone (vmcnt and expcnt left at their maximum).
__device__ inline void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (0x0 << 8) | (0x3 << 14)); }

template <int S>
struct Ring {
    bf16_t a[S][kTileRows * kBK];
    bf16_t b[S][kTileRows * kBK];
};

// Stage `kt`'s loads of this wave go to ring slot kt % S.  A row pointers
// advance by 64 elements per stage (row-major rows); B pointers by one
// 128 x 64 tile image (8192 elements).  issue_a / issue_b each send 4 loads.
constexpr int kTileElems = kTileRows * kBK;

template <int S>
__device__ inline void issue_a(Ring<S>& ring, const RowPtrs& A, int kt, int wave) {
    bf16_t* a = ring.a[kt % S] + wave * 32 * kBK;
    const int ka = kt * kBK;
    dma16(A.p0 + ka, a);
    dma16(A.p1 + ka, a + 8 * kBK);
    dma16(A.p2 + ka, a + 16 * kBK);
    dma16(A.p3 + ka, a + 24 * kBK);
}

template <int S>
__device__ inline void issue_b(Ring<S>& ring, const RowPtrs& B, int kt, int wave) {
    bf16_t* b = ring.b[kt % S] + wave * 32 * kBK;
    const int kb = kt * kTileElems;
    dma16(B.p0 + kb, b);
    dma16(B.p1 + kb, b + 8 * kBK);
    dma16(B.p2 + kb, b + 16 * kBK);
    dma16(B.p3 + kb, b + 24 * kBK);
}

// Wait until this wave's loads of stage kt have landed: the loads of the
// min(S-2, KT-1-kt) later stages (8 each) may stay in flight.
template <int S>
__device__ inline void wait_stage(int later) {
    if constexpr (S >= 4) {
        if (later >= 2) { wait_vm_lgkm0<16>(); return; }
    }
    if constexpr (S >= 3) {
        if (later >= 1) { wait_vm_lgkm0<8>(); return; }
    }
    wait_vm_lgkm0<0>();
}

// MFMA operands of one 16-k step: two A fragments (rows wm*64 + 32i) and two
// B fragments (rows bb0, bb1).
struct Frags {
    bf16x8_t a[2];
    bf16x8_t b[2];
};

__device__ inline void load_frags(Frags& f, const bf16_t* as, const bf16_t* bs, int kk, int lane, int wm,
                                  int bb0, int bb1) {
    const int chunk = kk * 2 + (lane >> 5);
#pragma unroll
    for (int i = 0; i < 2; ++i)
        f.a[i] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(as + swz(wm * 64 + i * 32 + (lane & 31), chunk)));
    f.b[0] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(bs + swz(bb0 + (lane & 31), chunk)));
    f.b[1] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(bs + swz(bb1 + (lane & 31), chunk)));
}

// B fragments go in the MFMA's first operand slot: the result is then the
// transposed tile, so each lane holds one token row (lane % 32) and, per
// accumulator register group, four consecutive output columns -- the shape
// the epilogue stores as 8-byte runs.
__device__ inline void mma(const Frags& f, f32x16_t (&acc)[2][2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma(f.b[j], f.a[i], acc[i][j]);
}

#define APS_PIN() __builtin_amdgcn_sched_barrier(0)

// acc[i][j] += A rows (wm*64 + 32i ..) x B rows (bb0/bb1 ..) over K = KT*64.
// Per stage: the LDS operand reads of step kk+1 are issued before the MFMAs
// of step kk (two fragment sets, ping-pong), and the next stage's 8 loads
// are spread between the MFMA groups; APS_PIN keeps that order.
template <int S>
__device__ inline void mainloop(Ring<S>& ring, const RowPtrs& A, const RowPtrs& B, int KT, int wave,
                                int lane, int wm, int bb0, int bb1, f32x16_t (&acc)[2][2]) {
#pragma unroll
    for (int s = 0; s < S - 1; ++s) {
        if (s < KT) {
            issue_a<S>(ring, A, s, wave);
            issue_b<S>(ring, B, s, wave);
        }
    }
    for (int kt = 0; kt < KT; ++kt) {
        const int later = (KT - 1 - kt) < (S - 2) ? (KT - 1 - kt) : (S - 2);
        wait_stage<S>(later);
        raw_barrier();
        const bool more = kt + S - 1 < KT;
        const bf16_t* as = ring.a[kt % S];
        const bf16_t* bs = ring.b[kt % S];
        Frags f0, f1;
        load_frags(f0, as, bs, 0, lane, wm, bb0, bb1);
        if (more) issue_a<S>(ring, A, kt + S - 1, wave);
        load_frags(f1, as, bs, 1, lane, wm, bb0, bb1);
        APS_PIN();
        mma(f0, acc);
        APS_PIN();
        if (more) issue_b<S>(ring, B, kt + S - 1, wave);
        load_frags(f0, as, bs, 2, lane, wm, bb0, bb1);
        APS_PIN();
        mma(f1, acc);
        APS_PIN();
        load_frags(f1, as, bs, 3, lane, wm, bb0, bb1);
        APS_PIN();
        mma(f0, acc);
        APS_PIN();
        mma(f1, acc);
    }
}

// Row (within the 128-row tile) and logical chunk of this lane's load in
// load instruction j: row 32*wave + 8j + lane/8 lands at physical chunk
// lane & 7, so it must fetch logical chunk (lane & 7) ^ ((row >> 1) & 7).
__device__ inline int dma_row(int wave, int j, int lane) { return wave * 32 + j * 8 + (lane >> 3); }
__device__ inline int dma_chunk(int wave, int j, int lane) {
    return (lane & 7) ^ ((dma_row(wave, j, lane) >> 1) & 7);
}

__device__ inline void zero_acc(f32x16_t (&acc)[2][2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][h][v] = 0.0f;
}

// ---------------------------------------------------------------------------
// Wide / tall blocks for the w1||w3 GEMM: one wave per SIMD, each wave owning
// a 64-row x 128-column MFMA tile (2 x 4 tiles of 32x32: 128 fp32
// accumulators per lane).  Per 32x32x16 step a wave reads 2 A + 4 B operand
// fragments (6 KB of LDS) for 8 MFMAs: 42.7 FLOP per LDS byte, against 32 for
// a 64x64 wave tile, which is what keeps the LDS (128 B/clk/CU) from being
// the bound.  A stage holds kStageRows = 384 tile rows of 64 k (48 KB): RA
// rows of A (token rows) followed by 384 - RA rows of B (packed w13 tile
// rows):
//   wide: RA = 128 -> 128 token rows x two column blocks (2 x (64 gate + 64
//         up)); waves (w & 1) pick the row half, (w >> 1) the column block;
//   tall: RA = 256 -> 256 token rows x one column block; wave w takes rows
//         64w..64w+63.
// Both shapes do the same MFMA work and move the same bytes per stage.  The
// work list holds every (128-row tile, column pair) as a wide block and, when
// F / 64 is odd, every (256-row tile, last column block) as a tall block, so
// the odd column block costs as much as a pair and the list stays about one
// block per CU (C2: 216 wide + 39 tall = 255 blocks).
constexpr int kStageRows = 384;
constexpr int kStageElems = kStageRows * kBK;  // 24576 bf16 = 48 KB
constexpr int kStages3 = 3;                    // 3 x 48 KB = 144 KB of LDS

struct Ring3 {
    bf16_t s[kStages3][kStageElems];
};

template <bool TALL>
struct UpShape {
    static constexpr int RA = TALL ? 256 : 128;  // A rows per stage
    static constexpr int NA = RA / 32;           // A slots per wave (8 rows x 4 waves per slot)
    static constexpr int NS = kStageRows / 32;   // 12 load slots per wave per stage
};

// Load slot s of wave w copies stage rows 32s + 8w .. +8 (1 KB).  A slots
// advance 64 elements per stage (row-major rows), B slots one 128 x 64 tile
// image (8192 elements).
struct Slots {
    const bf16_t* p[12];
};

template <bool TALL>
__device__ inline void issue_slots(bf16_t* stage, const Slots& sl, int kt, int wave, int lo, int hi) {
#pragma unroll
    for (int s = lo; s < hi; ++s) {
        const int64_t adv = s < UpShape<TALL>::NA ? static_cast<int64_t>(kt) * kBK
                                                 : static_cast<int64_t>(kt) * kTileElems;
        dma16(sl.p[s] + adv, stage + (32 * s + 8 * wave) * kBK);
    }
}

struct Frags6 {
    bf16x8_t a[2];
    bf16x8_t b[4];
};

__device__ inline void load_frags6(Frags6& f, const bf16_t* st, int kk, int lane, int aR, int bR) {
    const int chunk = kk * 2 + (lane >> 5);
#pragma unroll
    for (int i = 0; i < 2; ++i)
        f.a[i] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(st + swz(aR + i * 32 + (lane & 31), chunk)));
#pragma unroll
    for (int j = 0; j < 4; ++j)
        f.b[j] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(st + swz(bR + j * 32 + (lane & 31), chunk)));
}

__device__ inline void mma6(const Frags6& f, f32x16_t (&acc)[2][4]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma(f.b[j], f.a[i], acc[i][j]);
}

// acc[i][j] += stage rows aR + 32i (A) x stage rows bR + 32j (B) over
// K = KT * 64.  Three 48 KB stages.  The operand fragments of 16-k step g+1
// are read from LDS while the MFMAs of step g run (two fragment sets), and
// the stage hand-over sits between the MFMAs of the third and fourth steps
// of a stage: wait until stage kt+1 has landed (only stage kt+2 may still be
// in flight) and every read of stage kt is done, one s_barrier, read stage
// kt+1's first fragments, and only then issue stage kt's last MFMAs -- so the
// barrier and the first LDS latency of a stage hide behind MFMA work instead
// of stalling the SIMD.  The slot freed by that barrier (stage kt's) is
// refilled with stage kt+3 during the first three steps of stage kt+1.
template <bool TALL>
__device__ inline void mainloop3(Ring3& ring, const Slots& sl, int KT, int wave, int lane, int aR, int bR,
                                 f32x16_t (&acc)[2][4]) {
    issue_slots<TALL>(ring.s[0], sl, 0, wave, 0, 12);
    if (KT > 1) issue_slots<TALL>(ring.s[1], sl, 1, wave, 0, 12);
    if (KT > 2) issue_slots<TALL>(ring.s[2], sl, 2, wave, 0, 12);
    if (KT > 2) wait_vm_lgkm0<24>();
    else if (KT > 1) wait_vm_lgkm0<12>();
    else wait_vm_lgkm0<0>();
    raw_barrier();
    Frags6 fa, fb;
    load_frags6(fa, ring.s[0], 0, lane, aR, bR);
    int cur = 0;
    int prev = 2;            // slot of stage kt - 1, refilled with stage kt + 2
    for (int kt = 0; kt < KT; ++kt) {
        const bf16_t* st = ring.s[cur];
        const int nxt = cur == 2 ? 0 : cur + 1;
        const bool refill = kt >= 1 && kt + 2 < KT;  // stage kt + 2 goes to slot `prev`
        // Each step first waits for its own fragments (read one MFMA group
        // earlier), then issues the next step's reads, then its MFMAs: the
        // wait never covers the reads issued just before the MFMAs.  Stage
        // kt + 2's loads are spread over the first three steps.
        wait_lgkm0();
        load_frags6(fb, st, 1, lane, aR, bR);
        if (refill) issue_slots<TALL>(ring.s[prev], sl, kt + 2, wave, 0, 4);
        APS_PIN();
        mma6(fa, acc);
        APS_PIN();
        wait_lgkm0();
        load_frags6(fa, st, 2, lane, aR, bR);
        if (refill) issue_slots<TALL>(ring.s[prev], sl, kt + 2, wave, 4, 8);
        APS_PIN();
        mma6(fb, acc);
        APS_PIN();
        wait_lgkm0();
        load_frags6(fb, st, 3, lane, aR, bR);
        if (refill) issue_slots<TALL>(ring.s[prev], sl, kt + 2, wave, 8, 12);
        APS_PIN();
        mma6(fa, acc);
        APS_PIN();
        if (kt + 1 < KT) {
            // stage kt + 1 must have landed; stage kt + 2 may stay in flight
            if (kt + 2 < KT) wait_vm_lgkm0<12>();
            else wait_vm_lgkm0<0>();
            raw_barrier();
            load_frags6(fa, ring.s[nxt], 0, lane, aR, bR);
        } else {
            wait_lgkm0();
        }
        APS_PIN();
        mma6(fb, acc);
        APS_PIN();
        prev = cur;
        cur = nxt;
    }
}

// Work list of the w1||w3 kernel, expert by expert.  Expert e's rows form
// groups of 256 (two 128-row tiles); a group contributes, in order, the
// wide blocks of its row tiles (row tile major, F/128 column pairs each)
// and, when F / 64 is odd, one tall block (its 256 rows x the last column
// block).  Keeping a group's wide and tall blocks adjacent keeps their
// shared token rows in one XCD's L2 when XCD x takes the contiguous slice
// [x * per, (x + 1) * per) of the list (workgroup b runs on XCD b % 8).
struct UpTile {
    int expert, nb0;
    uint32_t m0, end;
    bool tall;
};

__device__ inline bool locate_up_tile(const uint32_t* __restrict__ offsets, int E, int F, UpTile& u) {
    const int lane = threadIdx.x & 63;
    const uint32_t lo = lane < E ? offsets[lane] : 0u;
    uint32_t hi = __shfl_down(lo, 1);
    if (lane == E - 1) hi = offsets[E];
    const uint32_t cnt = lane < E ? hi - lo : 0u;
    const int nblk = F / kBK, pairs = nblk / 2, odd = nblk & 1;
    const int r128 = static_cast<int>((cnt + 127) / 128);
    const int nb = pairs * r128 + odd * static_cast<int>((cnt + 255) / 256);  // blocks of this expert
    int incl = nb;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int v = __shfl_up(incl, d);
        if (lane >= d) incl += v;
    }
    const int total = __shfl(incl, 63);
    const int b = blockIdx.x;
    const int per = (total + kXcds - 1) / kXcds;
    const int l = b / kXcds;
    const int t = (b % kXcds) * per + l;
    if (l >= per || t >= total) return false;
    const uint64_t m = __ballot(lane < E && incl > t);
    const int e = __ffsll(static_cast<unsigned long long>(m)) - 1;
    const int before_incl = __shfl(incl, e > 0 ? e - 1 : 0);
    const int i = t - (e > 0 ? before_incl : 0);     // block index within expert e
    const int e_r128 = __shfl(r128, e);
    const int gsz = 2 * pairs + odd;                 // blocks of a full 256-row group
    const int g = i / gsz;
    const int r = i - g * gsz;
    const int nw = e_r128 - 2 * g < 2 ? e_r128 - 2 * g : 2;  // 128-row tiles in group g
    u.expert = e;
    u.end = __shfl(hi, e);
    const uint32_t e_lo = __shfl(lo, e);
    if (r < pairs * nw) {
        u.m0 = e_lo + static_cast<uint32_t>(2 * g + r / pairs) * 128u;
        u.nb0 = 2 * (r % pairs);
        u.tall = false;
    } else {
        u.m0 = e_lo + static_cast<uint32_t>(g) * 256u;
        u.nb0 = nblk - 1;
        u.tall = true;
    }
    return true;
}

// act[p][n] = silu(x[t] . w1[e][n]) * (x[t] . w3[e][n]),  t = assignment_rows[p]
template <bool TALL>
__device__ inline void ffn_up_block(Ring3& ring, const bf16_t* __restrict__ x,
                                    const uint32_t* __restrict__ assignment_rows,
                                    const bf16_t* __restrict__ w13, bf16_t* __restrict__ act, int H, int F,
                                    const UpTile& u) {
    using Sh = UpShape<TALL>;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int KT = H / kBK;
    // Load slots.  A: gathered token rows; positions past the expert's end
    // reuse its last row (a valid address; those rows are never stored).
    // B: rows of the packed tile images, copied verbatim (the images are
    // stored pre-swizzled, and RA is a multiple of 16 so the stage row and
    // the image row share their swizzle).
    Slots sl;
#pragma unroll
    for (int s = 0; s < 12; ++s) {
        const int row = 32 * s + 8 * wave + (lane >> 3);
        if (s < Sh::NA) {
            uint32_t p = u.m0 + row;
            p = p < u.end ? p : u.end - 1;
            const int chunk = (lane & 7) ^ ((row >> 1) & 7);
            sl.p[s] = x + static_cast<int64_t>(assignment_rows[p]) * H + chunk * 8;
        } else {
            const int rb = 32 * s + 8 * wave - Sh::RA;  // first B row of this slot
            const int cb = u.nb0 + rb / 128;
            sl.p[s] = w13 + (static_cast<int64_t>(u.expert) * (F / kBK) + cb) * 128 * static_cast<int64_t>(H) +
                      (rb % 128) * kBK + lane * 8;
        }
    }
    const int aR = TALL ? wave * 64 : (wave & 1) * 64;
    const int bR = Sh::RA + (TALL ? 0 : (wave >> 1) * 128);

    f32x16_t acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    mainloop3<TALL>(ring, sl, KT, wave, lane, aR, bR, acc);

    // Epilogue: SwiGLU in registers (B fragments 0,1 are gate columns 0..63
    // of the wave's column block, 2,3 the same up columns), the bf16 act tile
    // staged in the idle ring, then written as 16-byte row chunks.
    constexpr int kCols = TALL ? 64 : 128;   // act columns of the block tile
    constexpr int kPitch = kCols + 8;        // 16-byte aligned rows, banks staggered
    bf16_t* stage = ring.s[0];
    raw_barrier();
    const int cbase = TALL ? 0 : (wave >> 1) * 64;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int row = aR + i * 32 + (lane & 31);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int col = cbase + 32 * j + 8 * q + 4 * (lane >> 5);
                const u32x2_t v = {pack2_bf16(swiglu(acc[i][j][4 * q + 0], acc[i][j + 2][4 * q + 0]),
                                              swiglu(acc[i][j][4 * q + 1], acc[i][j + 2][4 * q + 1])),
                                   pack2_bf16(swiglu(acc[i][j][4 * q + 2], acc[i][j + 2][4 * q + 2]),
                                              swiglu(acc[i][j][4 * q + 3], acc[i][j + 2][4 * q + 3]))};
                *reinterpret_cast<u32x2_t*>(stage + row * kPitch + col) = v;
            }
    }
    wait_vm_lgkm0<0>();
    raw_barrier();
    constexpr int kChunks = kCols / 8;       // 16-byte chunks per row
#pragma unroll
    for (int c = 0; c < 8; ++c) {            // RA * kChunks = 2048 chunks
        const int id = tid + 256 * c;
        const int r = id / kChunks, cc = id % kChunks;
        const uint32_t p = u.m0 + r;
        if (p < u.end)
            *reinterpret_cast<u32x4_t*>(act + static_cast<int64_t>(p) * F + u.nb0 * kBK + cc * 8) =
                *reinterpret_cast<const u32x4_t*>(stage + r * kPitch + cc * 8);
    }
}

__global__ void __launch_bounds__(256, 1)
k_ffn_up_bf16(const bf16_t* __restrict__ x, const uint32_t* __restrict__ offsets,
              const uint32_t* __restrict__ assignment_rows, const bf16_t* __restrict__ w13,
              bf16_t* __restrict__ act, int H, int F, int E) {
    __shared__ __align__(16) Ring3 ring;
    UpTile u;
    if (!locate_up_tile(offsets, E, F, u)) return;
    if (u.tall) ffn_up_block<true>(ring, x, assignment_rows, w13, act, H, F, u);
    else ffn_up_block<false>(ring, x, assignment_rows, w13, act, H, F, u);
}

// ---------------------------------------------------------------------------
// y[p][n] = act[p] . w2[e][n]; block: 128 positions x 128 hidden columns.
template <int S, int OCC>
__global__ void __launch_bounds__(256, OCC)
k_ffn_down_bf16(const bf16_t* __restrict__ act, const uint32_t* __restrict__ offsets,
                const bf16_t* __restrict__ w2, bf16_t* __restrict__ y, int H, int F, int E) {
    __shared__ __align__(16) Ring<S> ring;

    int e, nb;
    uint32_t m0, end;
    if (!locate_tile(offsets, E, kDownBM, H / kDownBN, e, m0, end, nb)) return;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, lives in an SGPR
    const int wm = wave >> 1, wn = wave & 1;
    auto a_row = [&](int j) {
        uint32_t p = m0 + dma_row(wave, j, lane);
        p = p < end ? p : end - 1;
        return act + static_cast<int64_t>(p) * F + dma_chunk(wave, j, lane) * 8;
    };
    const RowPtrs A{a_row(0), a_row(1), a_row(2), a_row(3)};
    const bf16_t* wb = w2 + (static_cast<int64_t>(e) * (H / kDownBN) + nb) * 128 * static_cast<int64_t>(F);
    auto b_row = [&](int j) { return wb + (wave * 32 + j * 8) * kBK + lane * 8; };
    const RowPtrs B{b_row(0), b_row(1), b_row(2), b_row(3)};

    f32x16_t acc[2][2];
    zero_acc(acc);
    mainloop<S>(ring, A, B, F / kBK, wave, lane, wm, wn * 64, wn * 64 + 32, acc);

    // Epilogue: the 128 x 128 bf16 y tile staged in the (now idle) LDS ring,
    // then written out as 16-byte row chunks (256 contiguous bytes per row).
    constexpr int kPitch = kDownBN + 8;  // 272-byte rows: 16-byte aligned
    bf16_t* stage = ring.a[0];
    wait_vm_lgkm0<0>();
    raw_barrier();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int row = wm * 64 + i * 32 + (lane & 31);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int col = wn * 64 + j * 32 + 8 * q + 4 * (lane >> 5);
                const u32x2_t v = {pack2_bf16(acc[i][j][4 * q + 0], acc[i][j][4 * q + 1]),
                                   pack2_bf16(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3])};
                *reinterpret_cast<u32x2_t*>(stage + row * kPitch + col) = v;
            }
        }
    }
    wait_vm_lgkm0<0>();
    raw_barrier();
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int id = tid + 256 * c;   // 128 rows x 16 chunks of 16 bytes
        const int r = id >> 4, cc = id & 15;
        const uint32_t p = m0 + r;
        if (p < end)
            *reinterpret_cast<u32x4_t*>(y + static_cast<int64_t>(p) * H + static_cast<int64_t>(nb) * kDownBN + cc * 8) =
                *reinterpret_cast<const u32x4_t*>(stage + r * kPitch + cc * 8);
    }
}

}  // namespace

// Pipeline depth / occupancy variant (S stages of 32 KB; OCC blocks per CU).
// Default (2, 2): two stages per block, two blocks per CU (measured fastest
// at C2).  APS_FFN_VARIANT selects another for tuning runs: 1 = (4, 1),
// 2 = (3, 1).
static int ffn_variant() {
    static const int v = [] {
        const char* e = getenv("APS_FFN_VARIANT");
        return e ? atoi(e) : 0;
    }();
    return v;
}

hipError_t launch_ffn_up_bf16(const bf16_t* x, const uint32_t* offsets,
                              const uint32_t* assignment_rows, const bf16_t* w13,
                              bf16_t* act, int64_t rows, int hidden, int ffn, int experts,
                              hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hidden % kBK != 0 || ffn % kBK != 0) return hipErrorInvalidValue;
    const int nblk = ffn / kBK;
    const int64_t tiles = max_row_tiles(2 * rows, 128, experts) * (nblk / 2) +
                          ((nblk & 1) ? max_row_tiles(2 * rows, 256, experts) : 0);
    const dim3 grid(static_cast<unsigned>(ceil_div(tiles, kXcds) * kXcds));
    hipLaunchKernelGGL(k_ffn_up_bf16, grid, dim3(256), 0, s, x, offsets, assignment_rows, w13, act, hidden,
                       ffn, experts);
    return hipGetLastError();
}

hipError_t launch_ffn_down_bf16(const bf16_t* act, const uint32_t* offsets, const bf16_t* w2,
                                bf16_t* y, int64_t rows, int hidden, int ffn, int experts,
                                hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hidden % kDownBN != 0 || ffn % kBK != 0) return hipErrorInvalidValue;
    const int64_t tiles = max_row_tiles(2 * rows, kDownBM, experts) * (hidden / kDownBN);
    const dim3 grid(static_cast<unsigned>(ceil_div(tiles, kXcds) * kXcds));
    switch (ffn_variant()) {
        case 1:
            hipLaunchKernelGGL((k_ffn_down_bf16<4, 1>), grid, dim3(256), 0, s, act, offsets, w2, y, hidden, ffn,
                               experts);
            break;
        case 2:
            hipLaunchKernelGGL((k_ffn_down_bf16<3, 1>), grid, dim3(256), 0, s, act, offsets, w2, y, hidden, ffn,
                               experts);
            break;
        default:
            hipLaunchKernelGGL((k_ffn_down_bf16<2, 2>), grid, dim3(256), 0, s, act, offsets, w2, y, hidden, ffn,
                               experts);
    }
    return hipGetLastError();
}

}  // namespace aps
