// Grouped expert FFN on gfx950 bf16 MFMA (fp32 accumulate).
//
// Reference: k_moe_pair_silu_8x8 (src/tensor.cu:1838-1966) computes
// silu(x . w1^T) * (x . w3^T) for each expert's row range with the gather
// folded into the A load (assignment_rows), and k_moe_matmul_8x8
// (src/tensor.cu:1740-1836) multiplies by w2^T.  Both are fp32 SIMT GEMMs
// over a 128-row work list (src/tensor.cu:1333-1374).
//
// gfx950 design, shared by both GEMMs.
//  * One wave per SIMD; each wave owns a 64-row x 128-column output tile of
//    v_mfma_f32_32x32x16_bf16 (2 x 4 MFMA tiles, 128 fp32 accumulators per
//    lane).  Per 16-k step a wave reads 2 A + 4 B operand fragments (6 KB of
//    LDS) for 8 MFMAs: 42.7 FLOP per LDS byte, so LDS bandwidth (128 B/clk
//    per CU) stays below the MFMA rate.
//  * A block of 4 waves is "wide" (128 token rows x 2 column blocks) or
//    "tall" (256 token rows x 1 column block).  A column block is 128 B
//    rows: for w1||w3, 64 gate + the same 64 up rows (SwiGLU closes inside
//    each lane); for w2, 128 hidden columns.  Both shapes move 384 tile rows
//    x 64 k (48 KB) per stage and do the same MFMA work.
//  * Operands stream from global memory straight into a three-stage LDS
//    ring with global_load_lds_dwordx4 (no VGPR staging).  16-byte chunks
//    are XOR-swizzled for gfx950's 64-bank LDS so that neither the copies nor
//    the ds_read_b128 operand fetches conflict.
//  * w1||w3 and w2 are re-packed at registration into the swizzled 128 x 64
//    tile images the ring holds (launch_pack_*): a B row of a stage is 128
//    contiguous bytes, copied verbatim.
//  * The token gather of the w1||w3 GEMM is an index on the A load, as in
//    the reference: no permuted copy of x is ever written.
//  * The work list is built on the device from offsets[] (no host round
//    trip), expert by expert, and dealt to XCDs in contiguous slices so
//    operand reuse stays inside one L2; skewed experts simply own more
//    blocks.
#include "common.hpp"

namespace aps {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
// native vectors (not HIP's uint4 struct, whose copies become memcpy through
// a stack slot): 16 bytes = one ds_read_b128 / global_load_dwordx4
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kBK = 64;                 // k per LDS stage
constexpr int kTileElems = 128 * kBK;   // one packed 128 x 64 weight tile image
constexpr int kXcds = 8;
#ifndef APS_DOWN_TALL
#define APS_DOWN_TALL true
#endif

// Element offset of 16-byte chunk `chunk` (0..7) of stage row `row`.
// gfx950's LDS has 64 four-byte banks (a 256-byte bank row = two 128-byte
// stage rows) and serves a ds_read_b128 16 lanes at a time.  An MFMA
// operand fetch reads the same logical chunk from 16 consecutive rows, so the
// physical chunk is chunk ^ ((row >> 1) & 7): rows 2m and 2m+1 sit in the two
// halves of a bank row, and the eight pairs of a 16-row group get eight
// different chunks -- sixteen distinct 16-byte bank groups, no conflict.
__device__ inline int swz(int row, int chunk) { return row * kBK + ((chunk ^ ((row >> 1) & 7)) << 3); }

__device__ inline bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ inline f32x16_t mfma(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Two fp32 -> packed bf16, round to nearest even (one v_cvt_pk_bf16_f32).
__device__ inline uint32_t pack2_bf16(float lo, float hi) {
    bf16x2_t v;
    v[0] = static_cast<__bf16>(lo);
    v[1] = static_cast<__bf16>(hi);
    return __builtin_bit_cast(uint32_t, v);
}

// silu(g) * u for the bf16 path: fp32 math with the hardware exp2 and
// reciprocal (the result is rounded to bf16, far coarser than their error).
__device__ inline float swiglu(float g, float u) {
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

#define APS_GP(p) ((const __attribute__((address_space(1))) void*)(p))
#define APS_LP(p) ((__attribute__((address_space(3))) void*)(p))
#define APS_PIN() __builtin_amdgcn_sched_barrier(0)

// One direct-to-LDS copy: lane i writes LDS bytes [16i, 16i+16) of the
// wave-uniform 1 KB slot at lds_slot (eight 128-byte stage rows).
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

// s_waitcnt lgkmcnt(0) alone (vmcnt and expcnt left at their maximum).
__device__ inline void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (0x0 << 8) | (0x3 << 14)); }

// A raw s_barrier: __syncthreads() adds a workgroup fence, which drains every
// in-flight load (vmcnt(0)) and would serialise the ring.
__device__ inline void raw_barrier() { asm volatile("s_barrier" ::: "memory"); }

// ---------------------------------------------------------------------------
// Stage ring.  A stage holds kStageRows = 384 rows of 64 k: RA rows of A
// (token rows) followed by 384 - RA rows of B (packed weight tile rows).
constexpr int kStageRows = 384;
constexpr int kStageElems = kStageRows * kBK;  // 24576 bf16 = 48 KB
constexpr int kStages = 3;                     // 3 x 48 KB = 144 KB of LDS

struct Ring3 {
    bf16_t s[kStages][kStageElems];
};

template <bool TALL>
struct Shape {
    static constexpr int RA = TALL ? 256 : 128;  // A rows per stage
    static constexpr int NA = RA / 32;           // A slots per wave
};

// Load slot s (0..11) of wave w copies stage rows 32s + 8w .. +8 (1 KB).
// A slots advance 64 elements per stage (row-major rows), B slots one tile
// image (8192 elements).
struct Slots {
    const bf16_t* p[12];
};

template <bool TALL>
__device__ inline void issue_slots(bf16_t* stage, const Slots& sl, int kt, int wave, int lo, int hi) {
#pragma unroll
    for (int s = lo; s < hi; ++s) {
        const int64_t adv = s < Shape<TALL>::NA ? static_cast<int64_t>(kt) * kBK
                                               : static_cast<int64_t>(kt) * kTileElems;
        dma16(sl.p[s] + adv, stage + (32 * s + 8 * wave) * kBK);
    }
}

// Stage row and logical chunk of this lane in a load slot: lane i lands at
// physical chunk i & 7 of row 8 * (slot row group) + i / 8, so it fetches
// the logical chunk that swz() places there.
__device__ inline int slot_row(int s, int wave, int lane) { return 32 * s + 8 * wave + (lane >> 3); }
__device__ inline int slot_chunk(int row, int lane) { return (lane & 7) ^ ((row >> 1) & 7); }

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

// B fragments go in the MFMA's first operand slot: the result is then the
// transposed tile, so each lane holds one token row (lane % 32) and, per
// accumulator register group q = v / 4, the four consecutive output columns
// 8q + 4 * (lane / 32) .. +3 -- the shape the epilogues stage as 8-byte runs.
__device__ inline void mma6(const Frags6& f, f32x16_t (&acc)[2][4]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma(f.b[j], f.a[i], acc[i][j]);
}

// acc[i][j] += stage rows aR + 32i (A) x stage rows bR + 32j (B) over
// K = KT * 64.  The operand fragments of 16-k step g+1 are read from LDS
// while the MFMAs of step g run (two fragment sets); each step first waits
// for its own fragments and only then issues the next step's reads, so the
// compiler's LDS wait never covers reads issued just before the MFMAs.  The
// stage hand-over sits between the MFMAs of the third and fourth steps of a
// stage: wait until stage kt+1 has landed (only stage kt+2 may still be in
// flight) and every read of stage kt is done, one s_barrier, read stage
// kt+1's first fragments, and only then issue stage kt's last MFMAs -- the
// barrier and the first LDS latency of a stage hide behind MFMA work.  The
// slot freed by that barrier (stage kt's) is refilled with stage kt+3 during
// the first three steps of stage kt+1.
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

// ---------------------------------------------------------------------------
// Work list, expert by expert.  `nblk` column blocks per row (F/64 for
// w1||w3, H/128 for w2); pairs = nblk / 2 wide blocks per 128-row tile and,
// when nblk is odd, one tall block (256 rows x the last column block) per
// 256-row group.  Expert e's rows form 256-row groups; a group contributes,
// in order, the wide blocks of its two row tiles (row tile major) and then
// its tall block, so blocks sharing token rows are adjacent in the list and
// land in one XCD's L2 when XCD x takes the contiguous slice
// [x * per, (x + 1) * per) (workgroup b runs on XCD b % 8).  Every output
// position and column block is covered exactly once.
struct Tile {
    int expert, nb0;
    uint32_t m0, end;
    bool tall;
};

template <bool ALL_TALL>
__device__ inline bool locate_block(const uint32_t* __restrict__ offsets, int E, int nblk, Tile& u) {
    const int lane = threadIdx.x & 63;
    const uint32_t lo = lane < E ? offsets[lane] : 0u;
    uint32_t hi = __shfl_down(lo, 1);
    if (lane == E - 1) hi = offsets[E];
    const uint32_t cnt = lane < E ? hi - lo : 0u;
    // ALL_TALL: every column block as a tall block (no wide pairs).
    const int pairs = ALL_TALL ? 0 : nblk / 2, odd = ALL_TALL ? nblk : (nblk & 1);
    const int r128 = static_cast<int>((cnt + 127) / 128);
    int incl = pairs * r128 + odd * static_cast<int>((cnt + 255) / 256);  // blocks of this expert
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
    if (!ALL_TALL && r < pairs * nw) {
        const int pp = ALL_TALL ? 1 : pairs;     // pairs > 0 on this branch
        u.m0 = e_lo + static_cast<uint32_t>(2 * g + r / pp) * 128u;
        u.nb0 = 2 * (r % pp);
        u.tall = false;
    } else {
        u.m0 = e_lo + static_cast<uint32_t>(g) * 256u;
        u.nb0 = ALL_TALL ? r : nblk - 1;
        u.tall = true;
    }
    return true;
}

__device__ inline void zero_acc(f32x16_t (&acc)[2][4]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
}

// Stage rows of this wave's MFMA operands: A rows aR.. (64), B rows bR.. (128).
template <bool TALL>
__device__ inline int wave_a_row(int wave) { return TALL ? wave * 64 : (wave & 1) * 64; }
template <bool TALL>
__device__ inline int wave_b_row(int wave) { return Shape<TALL>::RA + (TALL ? 0 : (wave >> 1) * 128); }

// B slots: rows of the packed tile images of column blocks nb0 (and nb0+1
// for a wide block), copied verbatim -- the images are stored pre-swizzled,
// and RA is a multiple of 16, so a stage row and its image row share their
// swizzle.  `image0` is the first image of column block 0 of this expert.
template <bool TALL>
__device__ inline const bf16_t* b_slot(const bf16_t* image0, int64_t block_elems, int nb0, int s, int wave,
                                       int lane) {
    const int rb = 32 * s + 8 * wave - Shape<TALL>::RA;  // first B row of this slot
    return image0 + static_cast<int64_t>(nb0 + rb / 128) * block_elems + (rb % 128) * kBK + lane * 8;
}

// ---------------------------------------------------------------------------
// act[p][n] = silu(x[t] . w1[e][n]) * (x[t] . w3[e][n]),  t = assignment_rows[p]
template <bool TALL>
__device__ inline void ffn_up_block(Ring3& ring, const bf16_t* __restrict__ x,
                                    const uint32_t* __restrict__ assignment_rows,
                                    const bf16_t* __restrict__ w13, bf16_t* __restrict__ act, int H, int F,
                                    const Tile& u) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // A: gathered token rows; positions past the expert's end reuse its last
    // row (a valid address; those rows are never stored).
    Slots sl;
    const bf16_t* image0 = w13 + static_cast<int64_t>(u.expert) * (F / kBK) * 128 * static_cast<int64_t>(H);
#pragma unroll
    for (int s = 0; s < 12; ++s) {
        if (s < Shape<TALL>::NA) {
            const int row = slot_row(s, wave, lane);
            uint32_t p = u.m0 + row;
            p = p < u.end ? p : u.end - 1;
            sl.p[s] = x + static_cast<int64_t>(assignment_rows[p]) * H + slot_chunk(row, lane) * 8;
        } else {
            sl.p[s] = b_slot<TALL>(image0, 128 * static_cast<int64_t>(H), u.nb0, s, wave, lane);
        }
    }
    const int aR = wave_a_row<TALL>(wave), bR = wave_b_row<TALL>(wave);
    f32x16_t acc[2][4];
    zero_acc(acc);
    mainloop3<TALL>(ring, sl, H / kBK, wave, lane, aR, bR, acc);

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
    for (int c = 0; c < Shape<TALL>::RA * kChunks / 256; ++c) {
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
    Tile u;
    if (!locate_block<false>(offsets, E, F / kBK, u)) return;
    if (u.tall) ffn_up_block<true>(ring, x, assignment_rows, w13, act, H, F, u);
    else ffn_up_block<false>(ring, x, assignment_rows, w13, act, H, F, u);
}

// ---------------------------------------------------------------------------
// y[p][n] = act[p] . w2[e][n]; a column block is 128 hidden columns.
template <bool TALL>
__device__ inline void ffn_down_block(Ring3& ring, const bf16_t* __restrict__ act,
                                      const bf16_t* __restrict__ w2, bf16_t* __restrict__ y, int H, int F,
                                      const Tile& u) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    Slots sl;
    const bf16_t* image0 = w2 + static_cast<int64_t>(u.expert) * (H / 128) * 128 * static_cast<int64_t>(F);
#pragma unroll
    for (int s = 0; s < 12; ++s) {
        if (s < Shape<TALL>::NA) {
            const int row = slot_row(s, wave, lane);
            uint32_t p = u.m0 + row;
            p = p < u.end ? p : u.end - 1;
            sl.p[s] = act + static_cast<int64_t>(p) * F + slot_chunk(row, lane) * 8;
        } else {
            sl.p[s] = b_slot<TALL>(image0, 128 * static_cast<int64_t>(F), u.nb0, s, wave, lane);
        }
    }
    const int aR = wave_a_row<TALL>(wave), bR = wave_b_row<TALL>(wave);
    f32x16_t acc[2][4];
    zero_acc(acc);
    mainloop3<TALL>(ring, sl, F / kBK, wave, lane, aR, bR, acc);

    // Epilogue: the bf16 y tile staged in the idle ring (it spans the ring's
    // first two stages), then written as 16-byte row chunks.
    constexpr int kCols = TALL ? 128 : 256;  // y columns of the block tile
    constexpr int kPitch = kCols + 8;
    bf16_t* stage = ring.s[0];
    raw_barrier();
    const int cbase = TALL ? 0 : (wave >> 1) * 128;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int row = aR + i * 32 + (lane & 31);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int col = cbase + 32 * j + 8 * q + 4 * (lane >> 5);
                const u32x2_t v = {pack2_bf16(acc[i][j][4 * q + 0], acc[i][j][4 * q + 1]),
                                   pack2_bf16(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3])};
                *reinterpret_cast<u32x2_t*>(stage + row * kPitch + col) = v;
            }
    }
    wait_vm_lgkm0<0>();
    raw_barrier();
    constexpr int kChunks = kCols / 8;
#pragma unroll
    for (int c = 0; c < Shape<TALL>::RA * kChunks / 256; ++c) {
        const int id = tid + 256 * c;
        const int r = id / kChunks, cc = id % kChunks;
        const uint32_t p = u.m0 + r;
        if (p < u.end)
            *reinterpret_cast<u32x4_t*>(y + static_cast<int64_t>(p) * H + u.nb0 * 128 + cc * 8) =
                *reinterpret_cast<const u32x4_t*>(stage + r * kPitch + cc * 8);
    }
}

__global__ void __launch_bounds__(256, 1)
k_ffn_down_bf16(const bf16_t* __restrict__ act, const uint32_t* __restrict__ offsets,
                const bf16_t* __restrict__ w2, bf16_t* __restrict__ y, int H, int F, int E) {
    __shared__ __align__(16) Ring3 ring;
    Tile u;
    if (!locate_block<APS_DOWN_TALL>(offsets, E, H / 128, u)) return;
    if (u.tall) ffn_down_block<true>(ring, act, w2, y, H, F, u);
    else ffn_down_block<false>(ring, act, w2, y, H, F, u);
}

// Upper bound on the work-list length for A = 2 * rows positions.
int64_t max_blocks(int64_t rows, int nblk, int experts, bool all_tall) {
    if (all_tall) return max_row_tiles(2 * rows, 256, experts) * nblk;
    return max_row_tiles(2 * rows, 128, experts) * (nblk / 2) +
           ((nblk & 1) ? max_row_tiles(2 * rows, 256, experts) : 0);
}

}  // namespace

hipError_t launch_ffn_up_bf16(const bf16_t* x, const uint32_t* offsets,
                              const uint32_t* assignment_rows, const bf16_t* w13,
                              bf16_t* act, int64_t rows, int hidden, int ffn, int experts,
                              hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hidden % kBK != 0 || ffn % kBK != 0) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(ceil_div(max_blocks(rows, ffn / kBK, experts, false), kXcds) * kXcds));
    hipLaunchKernelGGL(k_ffn_up_bf16, grid, dim3(256), 0, s, x, offsets, assignment_rows, w13, act, hidden,
                       ffn, experts);
    return hipGetLastError();
}

hipError_t launch_ffn_down_bf16(const bf16_t* act, const uint32_t* offsets, const bf16_t* w2,
                                bf16_t* y, int64_t rows, int hidden, int ffn, int experts,
                                hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hidden % 128 != 0 || ffn % kBK != 0) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(ceil_div(max_blocks(rows, hidden / 128, experts, APS_DOWN_TALL), kXcds) * kXcds));
    hipLaunchKernelGGL(k_ffn_down_bf16, grid, dim3(256), 0, s, act, offsets, w2, y, hidden, ffn, experts);
    return hipGetLastError();
}

}  // namespace aps
