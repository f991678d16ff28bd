// Grouped expert FFN on gfx950 MFMA: bf16 (fp32 accumulate) and fp8 e4m3
// (fp32 accumulate, per-channel weight scales, per-row activation scales).
//
// Reference: k_moe_pair_silu_8x8 (src/tensor.cu:1838-1966) computes
// silu(x . w1^T) * (x . w3^T) for each expert's row range with the gather
// folded into the A load (assignment_rows), and k_moe_matmul_8x8
// (src/tensor.cu:1740-1836) multiplies by w2^T.  Both are fp32 SIMT GEMMs
// over a 128-row work list (src/tensor.cu:1333-1374).  The reference has no
// bf16 or fp8 path; their numerics are this library's (documented at each
// epilogue).
//
// gfx950 design, shared by both GEMMs and both formats.
//  * One wave per SIMD; each wave owns a 64-row x 128-column output tile of
//    32x32 MFMAs (2 x 4 tiles, 128 fp32 accumulators per lane).  Per MFMA
//    k step a wave reads 2 A + 4 B operand fragments from LDS for 8 MFMAs:
//    42.7 FLOP per LDS byte in bf16 (85 in fp8), against 32 for a 64x64
//    wave tile, so LDS bandwidth (128 B/clk per CU) stays below the MFMA rate.
//  * A block of 4 waves is "wide" (128 token rows x 2 column blocks) or
//    "tall" (256 token rows x 1 column block).  A column block is 128 B
//    rows: for w1||w3, 64 gate + the same 64 up rows (SwiGLU closes inside
//    each lane); for w2, 128 hidden columns.
//  * Stages are byte rows: a stage holds 384 rows of 128 bytes (48 KB) --
//    64 k of bf16 or 128 k of fp8.  Operands stream from global memory
//    straight into a three-stage LDS ring with global_load_lds_dwordx4 (no
//    VGPR staging).  16-byte chunks are XOR-swizzled for gfx950's 64-bank
//    LDS so that neither the copies nor the ds_read_b128 operand fetches
//    conflict.
//  * Weights are re-packed at registration into the swizzled 128-row x
//    128-byte tile images (16 KB) the ring holds (launch_pack_*): a B row of
//    a stage is 128 contiguous bytes, copied verbatim.
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
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
// native vectors (not HIP's uint4 struct, whose copies become memcpy through
// a stack slot): 16 bytes = one ds_read_b128 / global_load_dwordx4
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kRowBytes = 128;                 // one stage row: 8 chunks of 16 bytes
constexpr int kImageBytes = 128 * kRowBytes;   // one packed weight tile image
constexpr int kXcds = 8;
#ifndef APS_DOWN_TALL
#define APS_DOWN_TALL true
#endif

// Byte offset of 16-byte chunk `chunk` (0..7) of stage row `row`.  gfx950's
// LDS has 64 four-byte banks (a 256-byte bank row = two stage rows) and
// serves a ds_read_b128 16 lanes at a time.  An MFMA operand fetch reads the
// same logical chunk from 16 consecutive rows, so the physical chunk is
// chunk ^ ((row >> 1) & 7): rows 2m and 2m+1 sit in the two halves of a bank
// row, and the eight pairs of a 16-row group get eight different chunks --
// sixteen distinct 16-byte bank groups, no conflict.
__device__ inline int swz(int row, int chunk) { return row * kRowBytes + ((chunk ^ ((row >> 1) & 7)) << 4); }

// Two fp32 -> packed bf16, round to nearest even (one v_cvt_pk_bf16_f32).
__device__ inline uint32_t pack2_bf16(float lo, float hi) {
    bf16x2_t v;
    v[0] = static_cast<__bf16>(lo);
    v[1] = static_cast<__bf16>(hi);
    return __builtin_bit_cast(uint32_t, v);
}

// silu(g) * u for the MFMA paths: fp32 math with the hardware exp2 and
// reciprocal (the result is rounded to bf16, far coarser than their error).
__device__ inline float swiglu(float g, float u) {
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

#define APS_GP(p) ((const __attribute__((address_space(1))) void*)(p))
#define APS_LP(p) ((__attribute__((address_space(3))) void*)(p))
#define APS_PIN() __builtin_amdgcn_sched_barrier(0)

// One direct-to-LDS copy: lane i writes LDS bytes [16i, 16i+16) of the
// wave-uniform 1 KB slot at lds_slot (eight stage rows).
__device__ inline void dma16(const uint8_t* src, uint8_t* lds_slot) {
    __builtin_amdgcn_global_load_lds(APS_GP(src), APS_LP(lds_slot), 16, 0, 0);
}

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] |
// lgkmcnt[11:8] | vmcnt[5:4] at bits [15:14]); n must be a constant.
template <int N>
__device__ inline void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
}

// s_waitcnt lgkmcnt(n) alone.
template <int N>
__device__ inline void wait_lgkm_n() {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (N << 8) | (0x3 << 14));
}

// wait_vm_lgkm0<n> for a value n in {0, 4, ..., 20} known only after
// unrolling (the s_waitcnt operand must be an immediate); other values wait
// for everything.
__device__ inline void wait_vm_lgkm0_upto20(int n) {
    switch (n) {
        case 20: wait_vm_lgkm0<20>(); break;
        case 16: wait_vm_lgkm0<16>(); break;
        case 12: wait_vm_lgkm0<12>(); break;
        case 8: wait_vm_lgkm0<8>(); break;
        case 4: wait_vm_lgkm0<4>(); break;
        default: wait_vm_lgkm0<0>(); break;
    }
}

// wait_vm_lgkm0<n> for a value n in {0, 4, ..., 32} known only at run time.
__device__ inline void wait_vm_lgkm0_upto32(int n) {
    switch (n) {
        case 32: wait_vm_lgkm0<32>(); break;
        case 28: wait_vm_lgkm0<28>(); break;
        case 24: wait_vm_lgkm0<24>(); break;
        default: wait_vm_lgkm0_upto20(n); break;
    }
}

// s_waitcnt lgkmcnt(0) alone (vmcnt and expcnt left at their maximum).
__device__ inline void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (0x0 << 8) | (0x3 << 14)); }

// A raw s_barrier: __syncthreads() adds a workgroup fence, which drains every
// in-flight load (vmcnt(0)) and would serialise the ring.
__device__ inline void raw_barrier() { asm volatile("s_barrier" ::: "memory"); }

// ---------------------------------------------------------------------------
// Operand formats.  kSub MFMA k steps per 128-byte stage row; a fragment is
// one lane's share of a 32-row MFMA operand: lane l holds row l % 32 and the
// k half (l / 32) of the step, the same for A and B.
struct Bf16Fmt {
    static constexpr int kSub = 4;             // 32x32x16: 16 k = 32 bytes per step
    static constexpr int kElt = 2;
    typedef bf16x8_t frag_t;
    __device__ static frag_t load(const uint8_t* st, int row, int kk, int lane) {
        return __builtin_bit_cast(frag_t, *reinterpret_cast<const u32x4_t*>(st + swz(row, 2 * kk + (lane >> 5))));
    }
    // a fragment is one ds_read_b128; load_part(.., 0) is load()
    static constexpr int kParts = 1;
    __device__ static void load_part(frag_t& f, const uint8_t* st, int row, int kk, int lane, int) {
        f = load(st, row, kk, lane);
    }
    __device__ static f32x16_t mma(const frag_t& a, const frag_t& b, f32x16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    // The register-resident w2 kernel pins its operands: accumulators in
    // VGPRs, the resident act fragments (second operand) in AGPRs, which
    // the MFMA reads directly.  Left to the allocator, the 224 act registers
    // plus 128 accumulators overflow the VGPR file and every step shuffles
    // operands between the two files.
    static constexpr bool kPinned = true;
    // NOP: three wait states in the same statement first, for a VALU write
    // of an operand register that the compiler may place right before it
    // (the hazard recognizer does not look into inline asm; 2 are needed)
    template <bool NOP = false>
    __device__ static void mma_pinned(f32x16_t& c, const frag_t& b, const frag_t& a) {
        if constexpr (NOP) asm("s_nop 2\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(b), "a"(a));
        else asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(b), "a"(a));
    }
    // the first k step of a tile: c = b x a + 0 (no zeroed accumulators)
    template <bool NOP = false>
    __device__ static void mma_pinned_first(f32x16_t& c, const frag_t& b, const frag_t& a) {
        if constexpr (NOP) asm("s_nop 2\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(b), "a"(a));
        else asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(b), "a"(a));
    }
};

struct Fp8Fmt {
    static constexpr int kSub = 2;             // 32x32x64: 64 k = 64 bytes per step
    static constexpr int kElt = 1;
    typedef i32x8_t frag_t;
    __device__ static frag_t load(const uint8_t* st, int row, int kk, int lane) {
        const int c = 4 * kk + 2 * (lane >> 5);
        const i32x4_t lo = *reinterpret_cast<const i32x4_t*>(st + swz(row, c));
        const i32x4_t hi = *reinterpret_cast<const i32x4_t*>(st + swz(row, c + 1));
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
    // a fragment is two ds_read_b128 (its low and high 16 bytes), issued
    // separately by the interleaved main loop
    static constexpr int kParts = 2;
    __device__ static void load_part(frag_t& f, const uint8_t* st, int row, int kk, int lane, int part) {
        const int c = 4 * kk + 2 * (lane >> 5) + part;
        const i32x4_t v = *reinterpret_cast<const i32x4_t*>(st + swz(row, c));
        const i32x4_t lo = __builtin_shufflevector(f, f, 0, 1, 2, 3);
        const i32x4_t hi = __builtin_shufflevector(f, f, 4, 5, 6, 7);
        f = part == 0 ? __builtin_shufflevector(v, hi, 0, 1, 2, 3, 4, 5, 6, 7)
                      : __builtin_shufflevector(lo, v, 0, 1, 2, 3, 4, 5, 6, 7);
    }
    // e4m3 x e4m3 (format code 0 for both operands), unit scales
    __device__ static f32x16_t mma(const frag_t& a, const frag_t& b, f32x16_t c) {
        return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
    }
    // The register-resident w2 kernel pins its operands as for bf16:
    // accumulators in VGPRs, the resident act fragments in AGPRs, so that
    // the epilogue reads the accumulators without v_accvgpr_read (128 VALU
    // moves per column block, which add to the MFMA time on a SIMD).
    static constexpr bool kPinned = true;
    template <bool NOP = false>
    __device__ static void mma_pinned(f32x16_t& c, const frag_t& b, const frag_t& a) {
        if constexpr (NOP) asm("s_nop 2\n\tv_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, %0" : "+v"(c) : "v"(b), "a"(a));
        else asm("v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, %0" : "+v"(c) : "v"(b), "a"(a));
    }
    template <bool NOP = false>
    __device__ static void mma_pinned_first(f32x16_t& c, const frag_t& b, const frag_t& a) {
        if constexpr (NOP) asm("s_nop 2\n\tv_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, 0" : "=&v"(c) : "v"(b), "a"(a));
        else asm("v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, 0" : "=&v"(c) : "v"(b), "a"(a));
    }
};

// ---------------------------------------------------------------------------
// Stage ring.  A stage holds kStageRows = 384 rows of 128 bytes: RA rows of
// A (token rows) followed by 384 - RA rows of B (packed weight tile rows).
constexpr int kStageRows = 384;
constexpr int kStageBytes = kStageRows * kRowBytes;  // 48 KB
constexpr int kStages = 3;                           // 3 x 48 KB = 144 KB of LDS

struct Ring3 {
    uint8_t s[kStages][kStageBytes];
};

template <bool TALL>
struct Shape {
    static constexpr int RA = TALL ? 256 : 128;  // A rows per stage
    static constexpr int NA = RA / 32;           // A slots per wave
};

// Load slot s (0..11) of wave w copies stage rows 32s + 8w .. +8 (1 KB).
// A slots advance one 128-byte row chunk per stage, B slots one tile image.
struct Slots {
    const uint8_t* p[12];
};

template <bool TALL>
__device__ inline void issue_slots(uint8_t* stage, const Slots& sl, int kt, int wave, int lo, int hi) {
#pragma unroll
    for (int s = lo; s < hi; ++s) {
        const int64_t adv = s < Shape<TALL>::NA ? static_cast<int64_t>(kt) * kRowBytes
                                               : static_cast<int64_t>(kt) * kImageBytes;
        dma16(sl.p[s] + adv, stage + (32 * s + 8 * wave) * kRowBytes);
    }
}

// Stage row and logical chunk of this lane in a load slot: lane i lands at
// physical chunk i & 7 of row 8 * (slot row group) + i / 8, so it fetches
// the logical chunk that swz() places there.
__device__ inline int slot_row(int s, int wave, int lane) { return 32 * s + 8 * wave + (lane >> 3); }
__device__ inline int slot_chunk(int row, int lane) { return (lane & 7) ^ ((row >> 1) & 7); }

template <class Fmt>
struct Frags {
    typename Fmt::frag_t a[2];
    typename Fmt::frag_t b[4];
};

template <class Fmt>
__device__ inline void load_frags(Frags<Fmt>& f, const uint8_t* st, int kk, int lane, int aR, int bR) {
#pragma unroll
    for (int i = 0; i < 2; ++i) f.a[i] = Fmt::load(st, aR + i * 32 + (lane & 31), kk, lane);
#pragma unroll
    for (int j = 0; j < 4; ++j) f.b[j] = Fmt::load(st, bR + j * 32 + (lane & 31), kk, lane);
}

// B fragments go in the MFMA's first operand slot: the result is then the
// transposed tile, so each lane holds one token row (lane % 32) and, per
// accumulator register group q = v / 4, the four consecutive output columns
// 8q + 4 * (lane / 32) .. +3 -- the shape the epilogues stage as 8-byte runs.
template <class Fmt>
__device__ inline void mma_frags(const Frags<Fmt>& f, f32x16_t (&acc)[2][4]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = Fmt::mma(f.b[j], f.a[i], acc[i][j]);
}

// acc[i][j] += stage rows aR + 32i (A) x stage rows bR + 32j (B) over KT
// stages.  The operand fragments of MFMA step g+1 are read from LDS while
// the MFMAs of step g run (two fragment sets); each step first waits for its
// own fragments and only then issues the next step's reads, so the compiler's
// LDS wait never covers reads issued just before the MFMAs.  The stage
// hand-over sits before the MFMAs of a stage's last step: wait until stage
// kt+1 has landed (only stage kt+2 may still be in flight) and every read of
// stage kt is done, one s_barrier, read stage kt+1's first fragments, and
// only then issue stage kt's last MFMAs -- the barrier and the first LDS
// latency of a stage hide behind MFMA work.  The slot freed by that barrier
// (stage kt's) is refilled with stage kt+3 during stage kt+1's other steps.
template <bool TALL, class Fmt>
__device__ inline void mainloop3(Ring3& ring, const Slots& sl, int KT, int wave, int lane, int aR, int bR,
                                 f32x16_t (&acc)[2][4]) {
    constexpr int kSub = Fmt::kSub;
    static_assert(kSub % 2 == 0, "ping-pong needs an even step count");
    issue_slots<TALL>(ring.s[0], sl, 0, wave, 0, 12);
    if (KT > 1) issue_slots<TALL>(ring.s[1], sl, 1, wave, 0, 12);
    if (KT > 2) issue_slots<TALL>(ring.s[2], sl, 2, wave, 0, 12);
    if (KT > 2) wait_vm_lgkm0<24>();
    else if (KT > 1) wait_vm_lgkm0<12>();
    else wait_vm_lgkm0<0>();
    raw_barrier();
    Frags<Fmt> f[2];
    load_frags<Fmt>(f[0], ring.s[0], 0, lane, aR, bR);
    int cur = 0;
    int prev = 2;  // slot of stage kt - 1, refilled with stage kt + 2
    for (int kt = 0; kt < KT; ++kt) {
        const uint8_t* st = ring.s[cur];
        const int nxt = cur == 2 ? 0 : cur + 1;
        const bool refill = kt >= 1 && kt + 2 < KT;
#pragma unroll
        for (int s = 0; s + 1 < kSub; ++s) {
            wait_lgkm0();
            load_frags<Fmt>(f[(s + 1) & 1], st, s + 1, lane, aR, bR);
            if (refill) issue_slots<TALL>(ring.s[prev], sl, kt + 2, wave, 12 * s / (kSub - 1), 12 * (s + 1) / (kSub - 1));
            APS_PIN();
            mma_frags<Fmt>(f[s & 1], acc);
            APS_PIN();
        }
        if (kt + 1 < KT) {
            if (kt + 2 < KT) wait_vm_lgkm0<12>();
            else wait_vm_lgkm0<0>();
            raw_barrier();
            load_frags<Fmt>(f[0], ring.s[nxt], 0, lane, aR, bR);
        } else {
            wait_lgkm0();
        }
        APS_PIN();
        mma_frags<Fmt>(f[1], acc);
        APS_PIN();
        prev = cur;
        cur = nxt;
    }
}

// ---------------------------------------------------------------------------
// Work list, expert by expert.  `nblk` column blocks per row (F/64 for
// w1||w3, H/128 for w2); pairs = nblk / 2 wide blocks per 128-row tile and,
// when nblk is odd, one tall block (256 rows x the last column block) per
// 256-row group (ALL_TALL: every column block as a tall block).  Expert e's
// rows form 256-row groups; a group contributes, in order, the wide blocks
// of its two row tiles (row tile major) and then its tall block(s), so
// blocks sharing token rows are adjacent in the list and land in one XCD's
// L2 when XCD x takes the contiguous slice [x * per, (x + 1) * per)
// (workgroup b runs on XCD b % 8).  Every output position and column block
// is covered exactly once.
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
        const int pp = ALL_TALL ? 1 : pairs;         // pairs > 0 on this branch
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
// swizzle.  `image0` is the first image of column block 0 of this expert;
// a column block holds KT images.
template <bool TALL>
__device__ inline const uint8_t* b_slot(const uint8_t* image0, int64_t block_bytes, int nb0, int s, int wave,
                                        int lane) {
    const int rb = 32 * s + 8 * wave - Shape<TALL>::RA;  // first B row of this slot
    return image0 + static_cast<int64_t>(nb0 + rb / 128) * block_bytes + (rb % 128) * kRowBytes + lane * 16;
}

// Per-output-column scales of this lane for accumulator register group q of
// B fragment j: columns c0 + 32j + 8q + 4 * (lane / 32) .. +3.
__device__ inline float4 col_scales(const float* __restrict__ s, int c0, int j, int q, int lane) {
    return *reinterpret_cast<const float4*>(s + c0 + 32 * j + 8 * q + 4 * (lane >> 5));
}

// s_waitcnt lgkmcnt(n) for n in 0..15 known only after unrolling.
__device__ inline void wait_lgkm(int n) {
    switch (n) {
        case 15: wait_lgkm_n<15>(); break;
        case 14: wait_lgkm_n<14>(); break;
        case 13: wait_lgkm_n<13>(); break;
        case 12: wait_lgkm_n<12>(); break;
        case 11: wait_lgkm_n<11>(); break;
        case 10: wait_lgkm_n<10>(); break;
        case 9: wait_lgkm_n<9>(); break;
        case 8: wait_lgkm_n<8>(); break;
        case 7: wait_lgkm_n<7>(); break;
        case 6: wait_lgkm_n<6>(); break;
        case 5: wait_lgkm_n<5>(); break;
        case 4: wait_lgkm_n<4>(); break;
        case 3: wait_lgkm_n<3>(); break;
        case 2: wait_lgkm_n<2>(); break;
        case 1: wait_lgkm_n<1>(); break;
        default: wait_lgkm_n<0>(); break;
    }
}

// ---------------------------------------------------------------------------
// w1||w3 pieces.  A piece is a rectangle of one expert's act output: RA of
// its positions x a range of act columns, computed by one 4-wave block over
// the whole K.  The waves form a WM x WN grid; wave (wm, wn) = (w % WM,
// w / WM) owns MI 32-row A fragments and NJ 32-row B fragments: NJ / 2 gate
// and the same NJ / 2 up columns, so that SwiGLU closes inside each lane.
//   W: 128 rows x 2 column blocks  (WM 2, WN 2, MI 2, NJ 4)  stage 384 rows
//   T: 256 rows x 1 column block   (WM 4, WN 1, MI 2, NJ 4)  stage 384 rows
//   S: 128 rows x 1 column block   (WM 2, WN 2, MI 2, NJ 2)  stage 256 rows
//   Q: 128 rows x 1/2 column block (WM 4, WN 1, MI 1, NJ 2)  stage 192 rows
// A column block is 64 act columns (128 packed rows: 64 gate, then the same
// 64 up).  NJ = 2 waves own half h of one (32 gate + 32 up columns): S's
// wave wn takes half wn, a Q piece one half for all four waves.  A position
// always sits at the same lane and fragment row, a column at the same
// fragment column, and every output element accumulates the same MFMA
// sequence over k ascending, whichever piece computes it: the shapes are
// interchangeable bit for bit, and the scheduler below picks them freely.
enum PieceKind { kPieceW = 0, kPieceT = 1, kPieceS = 2, kPieceQ = 3 };

template <int KIND>
struct PShape;
template <>
struct PShape<kPieceW> { static constexpr int WM = 2, WN = 2, MI = 2, NJ = 4; };
template <>
struct PShape<kPieceT> { static constexpr int WM = 4, WN = 1, MI = 2, NJ = 4; };
template <>
struct PShape<kPieceS> { static constexpr int WM = 2, WN = 2, MI = 2, NJ = 2; };
template <>
struct PShape<kPieceQ> { static constexpr int WM = 4, WN = 1, MI = 1, NJ = 2; };

template <class Sh>
struct PDims {
    static constexpr int RA = Sh::WM * Sh::MI * 32;      // A rows (positions) per stage
    static constexpr int RB = Sh::WN * Sh::NJ * 32;      // B rows (packed weight rows) per stage
    static constexpr int NA = RA / 32;                   // A load slots per wave
    static constexpr int NS = (RA + RB) / 32;            // load slots per wave
    static constexpr int M = Sh::MI * Sh::NJ;            // MFMAs per step
    static constexpr int NR = Sh::MI + Sh::NJ;           // fragments per step
    static constexpr int kCols = Sh::WN * Sh::NJ / 2 * 32;  // act columns of the piece
    static_assert(RA + RB <= kStageRows, "stage fits the ring");
};

struct Piece {
    int kind, expert, cb0, half;   // half: the column-block half of a Q piece
    uint32_t m0, end;              // first position of the piece, expert's end
};

template <class Fmt, class Sh>
struct PFrags {
    typename Fmt::frag_t a[Sh::MI];
    typename Fmt::frag_t b[Sh::NJ];
};

// Part `part` of fragment o of a wave's step-kk operands, in the order the
// step's MFMAs first need them: a0, b0 .. b(NJ-1), a1 .. a(MI-1).
template <class Fmt, class Sh>
__device__ inline void pload(PFrags<Fmt, Sh>& f, const uint8_t* st, int kk, int lane, int aR, int bR, int o,
                             int part) {
    if (o == 0) Fmt::load_part(f.a[0], st, aR + (lane & 31), kk, lane, part);
    else if (o <= Sh::NJ) Fmt::load_part(f.b[o - 1], st, bR + (o - 1) * 32 + (lane & 31), kk, lane, part);
    else Fmt::load_part(f.a[o - Sh::NJ], st, aR + (o - Sh::NJ) * 32 + (lane & 31), kk, lane, part);
}

// MFMA q of a step: acc[q / NJ][q % NJ] += b[q % NJ] x a[q / NJ].
template <class Fmt, class Sh>
__device__ inline void pmma(const PFrags<Fmt, Sh>& f, f32x16_t (&acc)[Sh::MI][Sh::NJ], int q) {
    acc[q / Sh::NJ][q % Sh::NJ] = Fmt::mma(f.b[q % Sh::NJ], f.a[q / Sh::NJ], acc[q / Sh::NJ][q % Sh::NJ]);
}

// Copies of load slots [lo, hi) of stage kt (A slots advance one 128-byte
// row chunk per stage, B slots one 16 KB tile image).
template <class Sh>
__device__ inline void pissue(uint8_t* stage, const Slots& sl, int kt, int wave, int lo, int hi) {
#pragma unroll
    for (int s = lo; s < hi; ++s) {
        const int64_t adv = s < PDims<Sh>::NA ? static_cast<int64_t>(kt) * kRowBytes
                                              : static_cast<int64_t>(kt) * kImageBytes;
        dma16(sl.p[s] + adv, stage + (32 * s + 8 * wave) * kRowBytes);
    }
}

// One stage of the three-stage ring.  Every MFMA is issued with the fragment
// reads and stage copies of its shadow after it, so that the matrix pipe
// keeps working while the wave issues them (issued in a burst between groups
// of MFMAs, they left the pipe idle for about a quarter of each step).  A
// step s < kSub - 1 issues MFMA q and then: for q < MR, its share of the
// next step's fragments (MR = 3 of 8 MFMAs, fewer for small pieces); for
// q >= MR, its share of this step's refill copies (REFILL).  The compiler
// drains lgkmcnt before a step's first MFMA (it cannot count LDS reads past
// in-flight LDS DMA), so the reads go first, well before that wait.  The
// last step (the stage hand-over) issues MFMAs 0 .. MB - 1, waits for stage
// kt + 1 (vmcnt) and its own fragments, passes one s_barrier, and reads
// stage kt + 1's first fragments in the shadow of the remaining MFMAs.
// REFILL: this stage refills the slot of stage kt - 1 with stage kt + 2;
// NEXT: a stage kt + 1 exists; PEND: stage kt + 2's copies are in flight at
// the hand-over.  Only the issue order is chosen here: every output element
// accumulates its MFMAs in k order.
template <class Sh, class Fmt, bool REFILL, bool NEXT, bool PEND>
__device__ inline void pstage(Ring3& ring, const Slots& sl, int kt, int wave, int lane, int aR, int bR,
                              PFrags<Fmt, Sh> (&f)[2], f32x16_t (&acc)[Sh::MI][Sh::NJ]) {
    typedef PDims<Sh> D;
    constexpr int kSub = Fmt::kSub, P = Fmt::kParts;
    constexpr int M = D::M, NR = D::NR, NS = D::NS;
    constexpr int MR = M >= 8 ? 3 : (M >= 4 ? 2 : 1);   // MFMAs carrying the reads
    constexpr int MB = M >= 8 ? 2 : 1;                  // MFMAs before the hand-over barrier
    const uint8_t* st = ring.s[kt % 3];
#pragma unroll
    for (int s = 0; s < kSub; ++s) {
        const PFrags<Fmt, Sh>& fc = f[s & 1];
        PFrags<Fmt, Sh>& fn = f[(s + 1) & 1];
        if (s + 1 < kSub) {
            const int c0 = NS * s / (kSub - 1), nc = NS * (s + 1) / (kSub - 1) - c0;
#pragma unroll
            for (int q = 0; q < M; ++q) {
                pmma<Fmt, Sh>(fc, acc, q);
                APS_PIN();
                if (q < MR) {
#pragma unroll
                    for (int o = q * NR / MR; o < (q + 1) * NR / MR; ++o)
#pragma unroll
                        for (int part = 0; part < P; ++part) pload<Fmt, Sh>(fn, st, s + 1, lane, aR, bR, o, part);
                }
                if (REFILL) {
#pragma unroll
                    for (int c = 0; c < nc; ++c) {
                        const int qc = M > MR ? MR + c * (M - MR) / nc : M - 1;
                        if (qc == q) pissue<Sh>(ring.s[(kt + 2) % 3], sl, kt + 2, wave, c0 + c, c0 + c + 1);
                    }
                }
                APS_PIN();
            }
        } else {
#pragma unroll
            for (int q = 0; q < MB; ++q) {
                pmma<Fmt, Sh>(fc, acc, q);
                APS_PIN();
            }
            if (NEXT) {
                if (PEND) wait_vm_lgkm0<NS>();
                else wait_vm_lgkm0<0>();
                raw_barrier();
            } else {
                wait_lgkm0();
            }
            APS_PIN();
            const uint8_t* sn = ring.s[(kt + 1) % 3];
            constexpr int MRn = M - MB < 3 ? M - MB : 3;  // MFMAs carrying the next stage's reads
#pragma unroll
            for (int q = MB; q < M; ++q) {
                pmma<Fmt, Sh>(fc, acc, q);
                APS_PIN();
                if (NEXT && q - MB < MRn) {
                    const int k = q - MB;
#pragma unroll
                    for (int o = k * NR / MRn; o < (k + 1) * NR / MRn; ++o)
#pragma unroll
                        for (int part = 0; part < P; ++part) pload<Fmt, Sh>(f[0], sn, 0, lane, aR, bR, o, part);
                }
                APS_PIN();
            }
        }
    }
}

// acc += A x B over KT stages of the three-stage ring.  Stage kt lives in
// slot kt % 3; stages 0..2 are copied up front, stage kt + 2 during stage kt
// (1 <= kt <= KT - 3).
template <class Sh, class Fmt>
__device__ inline void pmainloop(Ring3& ring, const Slots& sl, int KT, int wave, int lane, int aR, int bR,
                                 f32x16_t (&acc)[Sh::MI][Sh::NJ]) {
    typedef PDims<Sh> D;
    constexpr int P = Fmt::kParts, NS = D::NS;
    pissue<Sh>(ring.s[0], sl, 0, wave, 0, NS);
    if (KT > 1) pissue<Sh>(ring.s[1], sl, 1, wave, 0, NS);
    if (KT > 2) pissue<Sh>(ring.s[2], sl, 2, wave, 0, NS);
    if (KT > 2) wait_vm_lgkm0<2 * NS>();
    else if (KT > 1) wait_vm_lgkm0<NS>();
    else wait_vm_lgkm0<0>();
    raw_barrier();
    PFrags<Fmt, Sh> f[2];
#pragma unroll
    for (int o = 0; o < D::NR; ++o)
#pragma unroll
        for (int part = 0; part < P; ++part) pload<Fmt, Sh>(f[0], ring.s[0], 0, lane, aR, bR, o, part);
    APS_PIN();
    if (KT == 1) {
        pstage<Sh, Fmt, false, false, false>(ring, sl, 0, wave, lane, aR, bR, f, acc);
        return;
    }
    if (KT > 2) pstage<Sh, Fmt, false, true, true>(ring, sl, 0, wave, lane, aR, bR, f, acc);
    else pstage<Sh, Fmt, false, true, false>(ring, sl, 0, wave, lane, aR, bR, f, acc);
    for (int kt = 1; kt + 2 < KT; ++kt) pstage<Sh, Fmt, true, true, true>(ring, sl, kt, wave, lane, aR, bR, f, acc);
    if (KT > 2) pstage<Sh, Fmt, false, true, false>(ring, sl, KT - 2, wave, lane, aR, bR, f, acc);
    pstage<Sh, Fmt, false, false, false>(ring, sl, KT - 1, wave, lane, aR, bR, f, acc);
}

// ---------------------------------------------------------------------------
// act[p][n] = silu(g) * u with, t = assignment_rows[p],
//   bf16: g = x[t] . w1[e][n], u = x[t] . w3[e][n]             (fp32 accumulate)
//   fp8 : g = (xq[t] . w1q[e][n]) * sx[t] * s1[e][n], u likewise with w3
//         (codes multiplied exactly, fp32 accumulate, then the two scales)
// act is stored as bf16.  One piece of shape Sh (see PShape).
template <class Sh, class Fmt>
__device__ inline void up_piece(Ring3& ring, const uint8_t* __restrict__ x, int64_t x_row_bytes,
                                const uint32_t* __restrict__ assignment_rows, const uint8_t* __restrict__ w13,
                                bf16_t* __restrict__ act, int H, int F, const float* __restrict__ sx,
                                const float* __restrict__ s1, const float* __restrict__ s3, const Piece& u) {
    typedef PDims<Sh> D;
    constexpr bool kFp8 = Fmt::kElt == 1;
    constexpr int MI = Sh::MI, NJ = Sh::NJ;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % Sh::WM, wn = wave / Sh::WM;
    const int KT = H * Fmt::kElt / kRowBytes;
    const int nblk = F / 64;
    // A slots: gathered token rows; positions past the expert's end reuse its
    // last row (a valid address; those rows are never stored).  B slots: 8
    // rows of a packed tile image, copied verbatim (the images are stored
    // pre-swizzled and every 32-row fragment group maps to 32 consecutive
    // image rows, so a stage row and its image row share their swizzle).
    Slots sl;
    const int64_t block_bytes = static_cast<int64_t>(KT) * kImageBytes;
    const uint8_t* image0 = w13 + static_cast<int64_t>(u.expert) * nblk * block_bytes;
#pragma unroll
    for (int s = 0; s < D::NS; ++s) {
        if (s < D::NA) {
            const int row = slot_row(s, wave, lane);
            uint32_t p = u.m0 + row;
            p = p < u.end ? p : u.end - 1;
            sl.p[s] = x + static_cast<int64_t>(assignment_rows[p]) * x_row_bytes + slot_chunk(row, lane) * 16;
        } else {
            const int rb = 32 * (s - D::NA) + 8 * wave;   // first B row of the slot
            int cb, ir;
            if (NJ == 4) {
                cb = u.cb0 + rb / 128;
                ir = rb % 128;
            } else {
                const int g = rb / 64, r = rb % 64, h = Sh::WN == 2 ? g : u.half;
                cb = u.cb0;
                ir = r < 32 ? 32 * h + r : 64 + 32 * h + (r - 32);
            }
            sl.p[s] = image0 + static_cast<int64_t>(cb) * block_bytes + ir * kRowBytes + lane * 16;
        }
    }
    const int aR = wm * MI * 32, bR = D::RA + wn * NJ * 32;
    f32x16_t acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    pmainloop<Sh, Fmt>(ring, sl, KT, wave, lane, aR, bR, acc);

    // Epilogue: scales (fp8), SwiGLU in registers (gate fragment j pairs with
    // up fragment j + NJ/2), the bf16 act tile staged in the idle ring, then
    // written as 16-byte row chunks.
    constexpr int kPitch = D::kCols + 8;      // elements; 16-byte aligned rows, banks staggered
    bf16_t* stage = reinterpret_cast<bf16_t*>(ring.s[0]);
    raw_barrier();
    const int hc = NJ == 4 ? 0 : (Sh::WN == 2 ? wn : u.half);  // column-block half (NJ = 2)
    const int gcol0 = (u.cb0 + (NJ == 4 ? wn : 0)) * 64 + (NJ == 4 ? 0 : 32 * hc);  // wave's first act column
    const int lcol0 = NJ == 4 ? wn * 64 : (Sh::WN == 2 ? wn * 32 : 0);             // ... within the piece
    const int c0 = u.expert * F + gcol0;      // its gate/up scale index (fp8)
    // fp8: every scale the epilogue needs is loaded first (the x row scales,
    // the w1 and w3 column scales), so that they cost one memory round
    // trip, not one per 4-column group
    typedef float ep_f32x4_t __attribute__((ext_vector_type(4)));
    float rsv[MI];
    ep_f32x4_t a1v[NJ / 2][4], a3v[NJ / 2][4];
    if constexpr (kFp8) {
        uint32_t ar[MI];
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            uint32_t p = u.m0 + aR + i * 32 + (lane & 31);
            p = p < u.end ? p : u.end - 1;
            ar[i] = assignment_rows[p];
        }
#pragma unroll
        for (int j = 0; j < NJ / 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int sc_at = c0 + 32 * j + 8 * q + 4 * (lane >> 5);
                a1v[j][q] = *reinterpret_cast<const ep_f32x4_t*>(s1 + sc_at);
                a3v[j][q] = *reinterpret_cast<const ep_f32x4_t*>(s3 + sc_at);
            }
#pragma unroll
        for (int i = 0; i < MI; ++i) rsv[i] = sx[ar[i]];
        // the values pass through empty asm statements: the compiler then
        // issues every load here (it had placed each pair of column-scale
        // loads next to its use, each followed by a vmcnt(0) wait)
#pragma unroll
        for (int j = 0; j < NJ / 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) asm volatile("" : "+v"(a1v[j][q]), "+v"(a3v[j][q]));
    }
#pragma unroll
    for (int i = 0; i < MI; ++i) {
        const int row = aR + i * 32 + (lane & 31);
        const float rs = kFp8 ? rsv[i] : 1.0f;
#pragma unroll
        for (int j = 0; j < NJ / 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float g[4], up[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    g[v] = acc[i][j][4 * q + v];
                    up[v] = acc[i][j + NJ / 2][4 * q + v];
                }
                if constexpr (kFp8) {
                    const ep_f32x4_t a1 = a1v[j][q], a3 = a3v[j][q];
                    g[0] = g[0] * rs * a1.x; g[1] = g[1] * rs * a1.y; g[2] = g[2] * rs * a1.z; g[3] = g[3] * rs * a1.w;
                    up[0] = up[0] * rs * a3.x; up[1] = up[1] * rs * a3.y; up[2] = up[2] * rs * a3.z; up[3] = up[3] * rs * a3.w;
                }
                const int col = lcol0 + 32 * j + 8 * q + 4 * (lane >> 5);
                const u32x2_t v = {pack2_bf16(swiglu(g[0], up[0]), swiglu(g[1], up[1])),
                                   pack2_bf16(swiglu(g[2], up[2]), swiglu(g[3], up[3]))};
                *reinterpret_cast<u32x2_t*>(stage + row * kPitch + col) = v;
            }
    }
    wait_vm_lgkm0<0>();
    raw_barrier();
    constexpr int kChunks = D::kCols / 8;     // 16-byte chunks per row
    const int acol = u.cb0 * 64 + (Sh::WN == 1 && NJ == 2 ? 32 * u.half : 0);  // piece's first act column
#pragma unroll
    for (int c = 0; c < D::RA * kChunks / 256; ++c) {
        const int id = tid + 256 * c;
        const int r = id / kChunks, cc = id % kChunks;
        const uint32_t p = u.m0 + r;
        if (p < u.end)
            *reinterpret_cast<u32x4_t*>(act + static_cast<int64_t>(p) * F + acol + cc * 8) =
                *reinterpret_cast<const u32x4_t*>(stage + r * kPitch + cc * 8);
    }
}

// ---------------------------------------------------------------------------
// Per-expert tile scheduler of the w1||w3 GEMM (the reference's work list,
// src/tensor.cu:1337-1374, with its grid sized by max_tall, :2846-2853),
// computed on the device from offsets[] by every block, identically.
//   Base list, expert by expert: each 256-row group of an expert's positions
// contributes the wide pieces W of its 128-row tiles (tile major) and, when
// the column-block count is odd, one piece for the last column block: T for
// the whole group, S when the group has at most 128 rows (the old tall
// block's empty half is never loaded).  Pieces sharing token rows or weights
// are adjacent in the list.
//   The grid is G persistent blocks (about one per CU, a multiple of the XCD
// count); workgroup b runs on XCD b % 8, as block l = b / 8 of its GX = G / 8.
// XCD x takes the contiguous slice [x * per, x * per + n) of the list (per =
// ceil(t / 8)), so blocks sharing token rows and weights share an L2, and
// deals it to its blocks in R = n / GX full rounds: round i gives block l
// the piece x * per + i * GX + l.  The r = n % GX pieces of the last round
// are split into s = 4, 2 or 1 pieces each (W -> 4 Q or 2 S, T -> 4 Q or
// 2 S by rows, S -> 2 Q), the largest s with r * s <= GX, and dealt the same
// way, siblings on adjacent blocks: a list just over one round then costs
// one W plus one Q per block instead of two rounds, and a small batch
// spreads over the whole chip.  Skewed experts simply own more of the list.
// Every block leaves after its at most R + 1 pieces.
struct UpSched {
    int E, nblk, pairs, odd, GX, l, first, R, r, s;
    uint32_t lo, hi;   // this lane's expert (lane = expert id): position range
    int r128, incl;    // its 128-row tiles; inclusive prefix count of base pieces
};

__device__ inline void up_sched(const uint32_t* __restrict__ offsets, int E, int nblk, UpSched& sc) {
    const int lane = threadIdx.x & 63;
    sc.E = E;
    sc.nblk = nblk;
    sc.pairs = nblk / 2;
    sc.odd = nblk & 1;
    sc.lo = lane < E ? offsets[lane] : 0u;
    sc.hi = __shfl_down(sc.lo, 1);
    if (lane == E - 1) sc.hi = offsets[E];
    const uint32_t cnt = lane < E ? sc.hi - sc.lo : 0u;
    sc.r128 = static_cast<int>((cnt + 127) / 128);
    int incl = sc.pairs * sc.r128 + sc.odd * static_cast<int>((cnt + 255) / 256);
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int v = __shfl_up(incl, d);
        if (lane >= d) incl += v;
    }
    sc.incl = incl;
    const int t = __shfl(incl, 63);
    sc.GX = static_cast<int>(gridDim.x) / kXcds;
    const int b = static_cast<int>(blockIdx.x), x = b % kXcds;
    sc.l = b / kXcds;
    const int per = (t + kXcds - 1) / kXcds;
    sc.first = x * per;
    const int last = sc.first + per < t ? sc.first + per : t;
    const int n = last > sc.first ? last - sc.first : 0;
    sc.R = n / sc.GX;
    sc.r = n - sc.R * sc.GX;
    sc.s = 4 * sc.r <= sc.GX ? 4 : (2 * sc.r <= sc.GX ? 2 : 1);
}

// Base piece t of the list (t < total).
__device__ inline Piece up_base(const UpSched& sc, int t) {
    const int lane = threadIdx.x & 63;
    const uint64_t m = __ballot(lane < sc.E && sc.incl > t);
    const int e = __ffsll(static_cast<unsigned long long>(m)) - 1;
    const int before = __shfl(sc.incl, e > 0 ? e - 1 : 0);
    const int i = t - (e > 0 ? before : 0);          // piece index within expert e
    const int e_r128 = __shfl(sc.r128, e);
    const int gsz = 2 * sc.pairs + sc.odd;           // pieces of a full 256-row group
    const int g = i / gsz, r = i - g * gsz;
    const int nw = e_r128 - 2 * g < 2 ? e_r128 - 2 * g : 2;  // 128-row tiles in group g
    Piece u;
    u.expert = e;
    u.end = __shfl(sc.hi, e);
    u.half = 0;
    const uint32_t e_lo = __shfl(sc.lo, e);
    if (r < sc.pairs * nw) {
        u.kind = kPieceW;
        u.m0 = e_lo + static_cast<uint32_t>(2 * g + r / sc.pairs) * 128u;
        u.cb0 = 2 * (r % sc.pairs);
    } else {
        u.kind = nw == 2 ? kPieceT : kPieceS;
        u.m0 = e_lo + static_cast<uint32_t>(g) * 256u;
        u.cb0 = sc.nblk - 1;
    }
    return u;
}

// Tail piece p of this XCD (p < r * s): sub-piece p % s of the slice's base
// piece R * GX + p / s.
__device__ inline bool up_tail(const UpSched& sc, int p, Piece& u) {
    const int sub = p % sc.s;
    u = up_base(sc, sc.first + sc.R * sc.GX + p / sc.s);
    if (sc.s == 1) return true;
    if (u.kind == kPieceW) {
        if (sc.s == 2) {
            u.kind = kPieceS;
            u.cb0 += sub;
        } else {
            u.kind = kPieceQ;
            u.cb0 += sub >> 1;
            u.half = sub & 1;
        }
    } else if (u.kind == kPieceT) {
        if (sc.s == 2) {
            u.kind = kPieceS;
            u.m0 += 128u * sub;
        } else {
            u.kind = kPieceQ;
            u.m0 += 128u * (sub >> 1);
            u.half = sub & 1;
        }
    } else {  // S: its two halves
        if (sub >= 2) return false;
        u.kind = kPieceQ;
        u.half = sub;
    }
    return u.m0 < u.end;
}

template <class Fmt>
__device__ inline void run_up_piece(Ring3& ring, const uint8_t* x, int64_t x_row_bytes, const uint32_t* arows,
                                    const uint8_t* w13, bf16_t* act, int H, int F, const float* sx,
                                    const float* s1, const float* s3, const Piece& u) {
    switch (u.kind) {
        case kPieceW: up_piece<PShape<kPieceW>, Fmt>(ring, x, x_row_bytes, arows, w13, act, H, F, sx, s1, s3, u); break;
        case kPieceT: up_piece<PShape<kPieceT>, Fmt>(ring, x, x_row_bytes, arows, w13, act, H, F, sx, s1, s3, u); break;
        case kPieceS: up_piece<PShape<kPieceS>, Fmt>(ring, x, x_row_bytes, arows, w13, act, H, F, sx, s1, s3, u); break;
        default: up_piece<PShape<kPieceQ>, Fmt>(ring, x, x_row_bytes, arows, w13, act, H, F, sx, s1, s3, u); break;
    }
}

template <class Fmt>
__global__ void __launch_bounds__(256, 1)
k_ffn_up(const uint8_t* __restrict__ x, int64_t x_row_bytes, const uint32_t* __restrict__ offsets,
         const uint32_t* __restrict__ assignment_rows, const uint8_t* __restrict__ w13, bf16_t* __restrict__ act,
         int H, int F, int E, const float* __restrict__ sx, const float* __restrict__ s1,
         const float* __restrict__ s3) {
    __shared__ __align__(16) Ring3 ring;
    UpSched sc;
    up_sched(offsets, E, F / 64, sc);
    // one call site, so that each piece shape is instantiated once
    for (int i = 0; i <= sc.R; ++i) {
        Piece u;
        if (i < sc.R) u = up_base(sc, sc.first + i * sc.GX + sc.l);
        else if (!(sc.l < sc.r * sc.s && up_tail(sc, sc.l, u))) break;
        u.kind = __builtin_amdgcn_readfirstlane(u.kind);
        u.expert = __builtin_amdgcn_readfirstlane(u.expert);
        u.cb0 = __builtin_amdgcn_readfirstlane(u.cb0);
        u.half = __builtin_amdgcn_readfirstlane(u.half);
        u.m0 = __builtin_amdgcn_readfirstlane(u.m0);
        u.end = __builtin_amdgcn_readfirstlane(u.end);
        if (i > 0) raw_barrier();  // the previous piece has read its staged tile out of the ring
        run_up_piece<Fmt>(ring, x, x_row_bytes, assignment_rows, w13, act, H, F, sx, s1, s3, u);
    }
}

// ---------------------------------------------------------------------------
// y[p][n], bf16, with
//   bf16: y = act[p] . w2[e][n]                               (fp32 accumulate)
//   fp8 : y = (actq[p] . w2q[e][n]) * sa[p] * s2[e][n]
// A rows are act_row_bytes apart; K = KT stages (fp8: F padded to 128).
template <bool TALL, class Fmt>
__device__ inline void ffn_down_block(Ring3& ring, const uint8_t* __restrict__ act, int64_t act_row_bytes,
                                      const uint8_t* __restrict__ w2, bf16_t* __restrict__ y, int H, int KT,
                                      const float* __restrict__ sa, const float* __restrict__ s2, const Tile& u) {
    constexpr bool kFp8 = Fmt::kElt == 1;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    Slots sl;
    const int64_t block_bytes = static_cast<int64_t>(KT) * kImageBytes;
    const uint8_t* image0 = w2 + static_cast<int64_t>(u.expert) * (H / 128) * block_bytes;
#pragma unroll
    for (int s = 0; s < 12; ++s) {
        if (s < Shape<TALL>::NA) {
            const int row = slot_row(s, wave, lane);
            uint32_t p = u.m0 + row;
            p = p < u.end ? p : u.end - 1;
            sl.p[s] = act + static_cast<int64_t>(p) * act_row_bytes + slot_chunk(row, lane) * 16;
        } else {
            sl.p[s] = b_slot<TALL>(image0, block_bytes, u.nb0, s, wave, lane);
        }
    }
    const int aR = wave_a_row<TALL>(wave), bR = wave_b_row<TALL>(wave);
    f32x16_t acc[2][4];
    zero_acc(acc);
    mainloop3<TALL, Fmt>(ring, sl, KT, wave, lane, aR, bR, acc);

    // Epilogue: scales (fp8), the bf16 y tile staged in the idle ring (it
    // spans the ring's first two stages), then written as 16-byte row chunks.
    constexpr int kCols = TALL ? 128 : 256;  // y columns of the block tile
    constexpr int kPitch = kCols + 8;
    bf16_t* stage = reinterpret_cast<bf16_t*>(ring.s[0]);
    raw_barrier();
    const int cbase = TALL ? 0 : (wave >> 1) * 128;
    const int c0 = u.expert * H + u.nb0 * 128 + cbase;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int row = aR + i * 32 + (lane & 31);
        float rs = 1.0f;
        if constexpr (kFp8) {
            uint32_t p = u.m0 + row;
            p = p < u.end ? p : u.end - 1;
            rs = sa[p];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float o[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) o[v] = acc[i][j][4 * q + v];
                if constexpr (kFp8) {
                    const float4 a = col_scales(s2, c0, j, q, lane);
                    o[0] = o[0] * rs * a.x; o[1] = o[1] * rs * a.y; o[2] = o[2] * rs * a.z; o[3] = o[3] * rs * a.w;
                }
                const int col = cbase + 32 * j + 8 * q + 4 * (lane >> 5);
                const u32x2_t v = {pack2_bf16(o[0], o[1]), pack2_bf16(o[2], o[3])};
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

template <class Fmt>
__global__ void __launch_bounds__(256, 1)
k_ffn_down(const uint8_t* __restrict__ act, int64_t act_row_bytes, const uint32_t* __restrict__ offsets,
           const uint8_t* __restrict__ w2, bf16_t* __restrict__ y, int H, int KT, int E,
           const float* __restrict__ sa, const float* __restrict__ s2) {
    __shared__ __align__(16) Ring3 ring;
    Tile u;
    if (!locate_block<APS_DOWN_TALL>(offsets, E, H / 128, u)) return;
    if (u.tall) ffn_down_block<true, Fmt>(ring, act, act_row_bytes, w2, y, H, KT, sa, s2, u);
    else ffn_down_block<false, Fmt>(ring, act, act_row_bytes, w2, y, H, KT, sa, s2, u);
}

// ---------------------------------------------------------------------------
// w2 with the act operand resident in registers.  K = F is short (448 bf16,
// 512 padded fp8), so a 256-position row tile of act fits the four waves'
// VGPRs (64 positions per wave: 224 VGPRs in bf16, 128 in fp8).  A block
// loads its row tile once and then streams w2 column blocks (128 hidden
// columns, KT images of 16 KB) through a four-slot LDS ring; every B byte
// feeds 256 positions (256 FLOP per LDS byte in bf16), so the loop is
// MFMA-bound where the streamed-A engine above is load-bound.  After a
// column block the tile is written through LDS as 16-byte row chunks while
// the ring already holds the next column block's first stages.
//   Work: each expert's positions form 256-row tiles; the H / 128 column
// blocks of a tile are split into S contiguous segments, S = the largest
// count that keeps tiles x S within the grid (about one block per CU).
// Logical blocks run expert-major, then segment, then tile, and XCD x takes
// a contiguous slice, so the blocks reading one w2 column range of an
// expert share an L2.
template <class Fmt>
struct DownAr;
template <>
struct DownAr<Bf16Fmt> { static constexpr int kKtMax = 7; };    // F <= 448
template <>
struct DownAr<Fp8Fmt> { static constexpr int kKtMax = 4; };     // F padded to <= 512

constexpr int kArRows = 256;                 // positions per block (4 waves x 64)
constexpr int kArSlots = 4;                  // w2 ring: 4 images of 16 KB
constexpr int kArPitch = 136;                // bf16 per staged y row (128 + 8)
constexpr int kArAStage = kArRows * kRowBytes;  // 32 KB: one act stage of the row tile

template <bool kFp8>
struct ArLds {
    uint8_t ring[kArSlots][kImageBytes];             // 64 KB
    uint8_t stage[kArRows * kArPitch * 2];           // 68 KB: the y tile, or two act stages
    float scl[kFp8 ? 32 * 128 : 4];                  // fp8: w2 column scales of the block's range
};

struct ArWork {
    int expert, nb0, nb1;
    uint32_t m0, end;
};

// Rows [lo, hi) of expert e in the list the kernel walks: positions of the
// routing plan (FOLD 0), or the dispatch's slot-ordered list, slot-0 rows
// (FOLD 1) or slot-1 rows (FOLD 2).
template <int FOLD>
__device__ inline bool locate_ar(const uint32_t* __restrict__ offsets, const uint32_t* __restrict__ slot1, int E,
                                 int NB, ArWork& u) {
    const int lane = threadIdx.x & 63;
    uint32_t lo = 0u, hi = 0u;
    if (lane < E) {
        lo = FOLD == 2 ? slot1[lane] : offsets[lane];
        hi = FOLD == 1 ? slot1[lane] : offsets[lane + 1];
    }
    const uint32_t cnt = lane < E ? hi - lo : 0u;
    const int r256 = static_cast<int>((cnt + kArRows - 1) / kArRows);
    int tiles = r256;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) tiles += __shfl_xor(tiles, d);
    if (tiles == 0) return false;
    const int G = static_cast<int>(gridDim.x);
    int S = G / tiles;
    S = S < 1 ? 1 : (S > NB ? NB : S);
    const int total = tiles * S;
    const int per = G / kXcds;
    const int b = blockIdx.x;
    const int t = (b % kXcds) * per + b / kXcds;
    if (t >= total) return false;
    int incl = r256 * S;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int v = __shfl_up(incl, d);
        if (lane >= d) incl += v;
    }
    const uint64_t m = __ballot(lane < E && incl > t);
    const int e = __ffsll(static_cast<unsigned long long>(m)) - 1;
    const int before = e > 0 ? __shfl(incl, e - 1) : 0;
    const int i = t - before;
    const int er = __shfl(r256, e);
    const int seg = i / er, tile = i - seg * er;
    // wave-uniform by construction; readfirstlane lets them live in SGPRs
    // (the y buffer resource must be scalar)
    u.expert = __builtin_amdgcn_readfirstlane(e);
    u.m0 = __builtin_amdgcn_readfirstlane(__shfl(lo, e) + static_cast<uint32_t>(tile) * kArRows);
    u.end = __builtin_amdgcn_readfirstlane(__shfl(hi, e));
    u.nb0 = __builtin_amdgcn_readfirstlane(seg * NB / S);
    u.nb1 = __builtin_amdgcn_readfirstlane((seg + 1) * NB / S);
    return true;
}

// y-tile stores through a buffer resource: rows past the expert's end fall
// outside num_records and the hardware drops them, so every thread issues
// the same number of stores (the vmcnt arithmetic below relies on it).
__device__ inline __amdgpu_buffer_rsrc_t y_rsrc(bf16_t* y, uint32_t m0, uint32_t end, int H, bool live) {
    const uint32_t rows = live ? (end - m0 < kArRows ? end - m0 : kArRows) : 0u;
    return __builtin_amdgcn_make_buffer_rsrc(y + static_cast<int64_t>(m0) * H, 0,
                                             static_cast<int>(rows * static_cast<uint32_t>(H) * 2u), 0x00020000);
}
// A buffer over `bytes` bytes of p (0: every access is dropped or reads 0).
__device__ inline __amdgpu_buffer_rsrc_t flat_rsrc(void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(p, 0, static_cast<int>(bytes), 0x00020000);
}
// Marks a row past the segment's end in the folded kernels' row tables
// (not an offset: every offset a buffer access takes stays below 2^31).
constexpr uint32_t kNoRow = 0xFFFFFFFFu;

// 16-byte chunks c0 .. c0 + N - 1 of this thread's share of the staged y
// tile: chunk c is tile row (tid + 256 c) / 16, column chunk (tid + 256 c) % 16.
template <int N>
__device__ inline void read_y_chunks(const bf16_t* stage, int c0, int tid, u32x4_t (&v)[N]) {
#pragma unroll
    for (int c = 0; c < N; ++c) {
        const int id = tid + 256 * (c0 + c);
        v[c] = *reinterpret_cast<const u32x4_t*>(stage + (id >> 4) * kArPitch + (id & 15) * 8);
    }
}
template <int N>
__device__ inline void write_y_chunks(__amdgpu_buffer_rsrc_t rs, int H, int nb, int c0, int tid, const u32x4_t (&v)[N]) {
#pragma unroll
    for (int c = 0; c < N; ++c) {
        const int id = tid + 256 * (c0 + c);
        __builtin_amdgcn_raw_buffer_store_b128(v[c], rs, (id >> 4) * H * 2 + nb * 256 + (id & 15) * 16, 0, 0);
    }
}

// The folded combine's rows.  rowoff[c] is the byte offset of this thread's
// chunk row c (tile row tid / 16 + 16 c) in a [T][H] bf16 array, token x
// 2H, or the array's size past the segment's end; tok_off adds the chunk's
// column (below 2^20), so a row past the end lands past the array, out of
// range of its buffer, and every offset stays below 2^31 (T H 2 + 2^20 <
// 2^31): the buffer range check drops such accesses, while offsets with bit
// 31 set must not be relied on to be dropped.
__device__ inline uint32_t tok_off(uint32_t rowoff, int nb, int tid) {
    return rowoff + static_cast<uint32_t>((nb * 128 + (tid & 15) * 8) * 2);
}
// The staged y tile's bytes (row pitch kArPitch bf16) as 17 direct-to-LDS
// copies per thread: copy i of thread tid fills stage bytes P = 4096 i +
// 16 tid, i.e. row P / 272 at byte P % 272.  kYaCopies covers 256 rows.
constexpr int kYaCopies = (kArRows * kArPitch * 2 + 4095) / 4096;
static_assert(kArPitch * 2 % 16 == 0, "16-byte copies tile a staged row");
// 4 bf16 of a and of b (u32x2 each): (0 + 0.5 a) + 0.5 b element-wise,
// rounded to bf16, as two FMAs: t = fma(b, 0.5, 0) is 0.5 b with -0 made +0
// (exact), then fma(a, 0.5, t) rounds 0.5 a + t once.  0.5 v is exact for a
// bf16 v, so this equals the reference's two rounded adds for every input
// pair, signed zeros included (the reference never yields -0: its first add
// turns -0 into +0; here t does, and a -0 first term meets +0 or a nonzero).
__device__ inline float combine_fma(float a, float b) { return __fmaf_rn(a, 0.5f, __fmaf_rn(b, 0.5f, 0.0f)); }
__device__ inline u32x2_t combine4_bf16(u32x2_t a, u32x2_t b) {
    float o[4];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        o[2 * k] = combine_fma(__uint_as_float(a[k] << 16), __uint_as_float(b[k] << 16));
        o[2 * k + 1] = combine_fma(__uint_as_float(a[k] & 0xFFFF0000u), __uint_as_float(b[k] & 0xFFFF0000u));
    }
    return u32x2_t{pack2_bf16(o[0], o[1]), pack2_bf16(o[2], o[3])};
}

// s_waitcnt vmcnt(n) lgkmcnt(0) for any n in 0 .. 47 known at run time.
template <int N>
__device__ inline void wait_vm_lgkm0_table(int n) {
    if constexpr (N < 0) {
        wait_vm_lgkm0<0>();
    } else {
        if (n == N) wait_vm_lgkm0<N>();
        else wait_vm_lgkm0_table<N - 1>(n);
    }
}
__device__ inline void wait_vm_lgkm0_n(int n) {
    if (n >= 47) wait_vm_lgkm0<47>();
    else wait_vm_lgkm0_table<46>(n);
}

// KT (k stages of 128 bytes) is a template argument so that the resident act
// fragments take exactly KT x 2 x kSub registers.  With KT >= 4 (the
// production shapes: F = 448 bf16, 512 fp8) the y tile of column block u-1
// leaves during the first four k stages of column block u, 4 chunks per
// stage, so the stores stream under MFMA work instead of stalling the ring.
//
// Schedule.  B fragments are read two MFMA steps ahead (three register
// sets).  Stage g+1's ring barrier (stage_ready) sits at step kSub-2 of stage
// g, just before its first fragments are read, and refills the slot of
// stage g-1 with stage g+3... (g+1)+2.  Per step: wait for this step's
// fragments, [barrier], [read this step's share of the staged y tile],
// read the fragments of step + 2, MFMAs, [store the y share].
//
// FOLD (the fused forward's combine, KT >= 4, bf16 output): the kernel walks
// one slot of the dispatch's slot-ordered lists (act rows gathered through
// slot_rows, outputs scattered to token rows).  FOLD 1 stores each slot-0
// row's bf16 output row to ya[token] (y is ya).  FOLD 2 (fp8) combines each
// slot-1 row with it into out[token] = (0 + 0.5 ya) + 0.5 y, the reference's
// combine: it stores the previous tile in k stages 0 and 1 (8 chunks each),
// which frees the stage; at k stage 2 it copies its own tile's ya rows into
// the stage (direct to LDS, in the stage's layout), and the epilogue
// combines each value in place.
template <class Fmt, int KT, int FOLD = 0>
__global__ void __launch_bounds__(256, 1)
k_ffn_down_ar(const uint8_t* __restrict__ act, int64_t act_row_bytes, const uint32_t* __restrict__ offsets,
              const uint8_t* __restrict__ w2, bf16_t* __restrict__ y, int H, int E,
              const float* __restrict__ sa, const float* __restrict__ s2, const uint32_t* __restrict__ slot1,
              const uint32_t* __restrict__ slot_rows, const uint32_t* __restrict__ slot_tokens,
              bf16_t* __restrict__ out, int64_t tokens) {
    constexpr bool kFp8 = Fmt::kElt == 1;
    constexpr bool kOverlap = KT >= 4;
    static_assert(FOLD == 0 || kOverlap, "the folded combine needs the overlapped stores");
    static_assert(FOLD != 2 || (kFp8 && KT == 4), "the folded combine's schedule is fp8's, four k stages");
    constexpr int KTM = KT;
    constexpr int kSub = Fmt::kSub;
    constexpr int kLoads = kFp8 ? 8 : 4;       // ds_read_b128 per fragment set
    constexpr int kChunks = FOLD == 2 ? 8 : 4;  // staged chunks stored per storing k stage
    static_assert(kSub >= 2, "two steps per stage");
    __shared__ __align__(16) ArLds<kFp8> lds;
    ArWork u;
    if (!locate_ar<FOLD>(offsets, slot1, E, H / 128, u)) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int aR = wave * 64;
    const int NB = H / 128;
    const int nunits = u.nb1 - u.nb0;
    const int nstages = nunits * KT;
    bf16_t* stage = reinterpret_cast<bf16_t*>(lds.stage);
    // FOLD 0: y tile rows m0 .. m0 + 255 (contiguous); FOLD 1 / 2: [T][H]
    // bf16 arrays (ya, out) addressed per row through rowoff[]
    const uint32_t tbytes = static_cast<uint32_t>(tokens) * static_cast<uint32_t>(H) * 2u;
    const __amdgpu_buffer_rsrc_t ys = FOLD == 0 ? y_rsrc(y, u.m0, u.end, H, true)
                                               : flat_rsrc(FOLD == 1 ? y : out, tbytes);
    const __amdgpu_buffer_rsrc_t ynull = FOLD == 0 ? y_rsrc(y, u.m0, u.end, H, false) : flat_rsrc(y, 0u);
    uint32_t rowoff[16];
    uint32_t yaoff[FOLD == 2 ? kYaCopies : 1];   // FOLD 2: ya source of each stage copy (kNoRow: none)
    if constexpr (FOLD != 0) {
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            const uint32_t q = u.m0 + static_cast<uint32_t>((tid >> 4) + 16 * c);
            const uint32_t tk = q < u.end ? slot_tokens[q] : kNoRow;
            rowoff[c] = tk < static_cast<uint32_t>(tokens) ? tk * static_cast<uint32_t>(2 * H) : tbytes;
        }
    }
    if constexpr (FOLD == 2) {
#pragma unroll
        for (int i = 0; i < kYaCopies; ++i) {
            const uint32_t P = 4096u * i + 16u * tid;
            const uint32_t row = P / (kArPitch * 2), b = P % (kArPitch * 2);
            const uint32_t q = u.m0 + row;
            uint32_t tk = row < kArRows && b < 256u && q < u.end ? slot_tokens[q] : kNoRow;
            yaoff[i] = tk < static_cast<uint32_t>(tokens) ? tk * static_cast<uint32_t>(2 * H) + b : kNoRow;
        }
    }
    // act row (plan position) of list entry q
    auto act_pos = [&](uint32_t q) -> uint32_t {
        q = q < u.end ? q : u.end - 1;
        if constexpr (FOLD == 0) return q;
        const uint32_t p = slot_rows[q];
        const uint32_t amax = 2u * static_cast<uint32_t>(tokens) - 1u;
        return p < amax ? p : amax;
    };

    // w2 ring: stage g = (unit g / KT, k stage g % KT); wave w copies bytes
    // [4 KB w, 4 KB w + 4 KB) of the 16 KB image, verbatim (pre-swizzled).
    const uint8_t* bsrc = w2 + (static_cast<int64_t>(u.expert) * NB + u.nb0) * KT * kImageBytes + wave * 4096 + lane * 16;
    auto issue_b = [&](int g) {
        const uint8_t* src = bsrc + static_cast<int64_t>(g) * kImageBytes;
        uint8_t* dst = lds.ring[g % kArSlots] + wave * 4096;
#pragma unroll
        for (int c = 0; c < 4; ++c) dma16(src + c * 1024, dst + c * 1024);
    };
    // FOLD 2: column block nb's ya rows into the stage (rows past the
    // segment read ya row 0 into rows whose results are dropped)
    auto issue_ya = [&](int nb) {
#pragma unroll
        for (int i = 0; i < kYaCopies; ++i) {
            const uint32_t off = yaoff[i] == kNoRow ? 0u : yaoff[i] + static_cast<uint32_t>(nb * 256);
            dma16(reinterpret_cast<const uint8_t*>(y) + off, lds.stage + 4096 * i + 1024 * wave);
        }
    };
    // VMEM operations issued at stage x (global index, x = unit x / KT, k
    // stage x % KT): staged-chunk stores (k stages 0..3, FOLD 2: 0..1) and
    // FOLD 2's stage copies (k stage 2).  Unit 0 has no previous tile: FOLD 0
    // issues its stores to a null buffer (same count at every unit), the
    // folded kernels issue none (the counts below follow).
    auto has_st = [](int k) { return kOverlap && (k + KTM) % KTM < (FOLD == 2 ? 2 : 4); };
    auto vm_at = [&](int x) {
        const bool st = has_st(x % KTM) && (FOLD == 0 || x >= KTM);
        return (st ? kChunks : 0) + (FOLD == 2 && x % KTM == 2 ? kYaCopies : 0);
    };
    // Stage g (k stage kt) landed for every wave.  Issued after stage g's
    // copies (at stage_ready(g-2)): stage g+1's copies, if any, and the
    // operations of k stages kt-2, kt-1 (bf16: the stores of a stage precede
    // its stage_ready) or kt-3, kt-2 (fp8: they follow it).  Stages 0..2
    // wait for everything.  Then stage g-2's slot takes stage g+2.
    auto stage_ready = [&](int g, int kt) {
        const int later = g + 1 < nstages ? 1 : 0;
        const int kS = g < 3 ? 0 : (kFp8 ? vm_at(g - 2) + vm_at(g - 3) : vm_at(g - 1) + vm_at(g - 2));
        if constexpr (FOLD == 2) wait_vm_lgkm0_n(g < 3 ? 0 : 4 * later + kS);
        else wait_vm_lgkm0_upto20(g < 3 ? 0 : 4 * later + kS);
        raw_barrier();
        if (g + 2 < nstages) issue_b(g + 2);
    };
    // fp8 scales: the block's w2 column scales into LDS, its 2 x 32 row scales per lane
    float rs[2] = {1.0f, 1.0f};
    if constexpr (kFp8) {
        const float* src = s2 + static_cast<int64_t>(u.expert) * H + u.nb0 * 128;
        for (int t = tid; t < nunits * 32; t += 256)
            *reinterpret_cast<float4*>(lds.scl + 4 * t) = *reinterpret_cast<const float4*>(src + 4 * t);
#pragma unroll
        for (int i = 0; i < 2; ++i) rs[i] = sa[act_pos(u.m0 + aR + 32 * i + (lane & 31))];
    }

    // ---- the row tile of act into registers, one 32 KB stage at a time ----
    // Four act slots, so that four stages are in flight: slots 0 and 1 are
    // the w2 ring (two images each), slots 2 and 3 the y stage.  Stage kt
    // uses slot kt % 4; once it is read, the slot takes stage kt + 4.  The w2
    // ring's first two stages are copied once the ring's act slot 0 has been
    // read for the last time (act stage kt0).
    typename Fmt::frag_t areg[KTM][2][kSub];
    {
        const uint8_t* asrc[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int row = slot_row(s, wave, lane);
            asrc[s] = act + static_cast<int64_t>(act_pos(u.m0 + row)) * act_row_bytes + slot_chunk(row, lane) * 16;
        }
        auto aslot = [&](int kt) -> uint8_t* {
            const int j = kt & 3;
            return j < 2 ? &lds.ring[0][0] + j * kArAStage : lds.stage + (j - 2) * kArAStage;
        };
        auto issue_a = [&](int kt) {
            uint8_t* st = aslot(kt);
#pragma unroll
            for (int s = 0; s < 8; ++s) dma16(asrc[s] + kt * kRowBytes, st + (32 * s + 8 * wave) * kRowBytes);
        };
        constexpr int kt0 = 4 * ((KT - 1) / 4);        // the last act stage in slot 0
        const int nbq = nstages < 2 ? nstages : 2;     // w2 stages copied after it
#pragma unroll
        for (int kt = 0; kt < (KT < 4 ? KT : 4); ++kt) issue_a(kt);
#pragma unroll
        for (int kt = 0; kt < KTM; ++kt) {
            if (kt < KT) {
                // copies issued after act stage kt: act stages kt+1 .. min(KT-1, kt+3)
                // (8 per wave each) and, past kt0, the w2 stages (4 each)
                const int a_after = (KT - 1 < kt + 3 ? KT - 1 : kt + 3) - kt;
                wait_vm_lgkm0_upto32(8 * a_after + (kt > kt0 ? 4 * nbq : 0));
                raw_barrier();
                const uint8_t* st = aslot(kt);
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int kk = 0; kk < kSub; ++kk) areg[kt][i][kk] = Fmt::load(st, aR + 32 * i + (lane & 31), kk, lane);
                wait_lgkm0();
                raw_barrier();  // slot kt % 4 is free; the last barrier frees the y stage and the ring
                if (kt + 4 < KT) issue_a(kt + 4);
                if (kt == kt0) {
                    if (nstages > 0) issue_b(0);
                    if (nstages > 1) issue_b(1);
                }
            }
        }
    }

    typename Fmt::frag_t bf[3][4];
    auto load_b = [&](typename Fmt::frag_t (&f)[4], int g, int kk) {
#pragma unroll
        for (int j = 0; j < 4; ++j) f[j] = Fmt::load(lds.ring[g % kArSlots], 32 * j + (lane & 31), kk, lane);
    };
    if (nstages > 0) stage_ready(0, 0);
    for (int ui = 0; ui < nunits; ++ui) {
        const int nb = u.nb0 + ui;
        const int g0 = ui * KT;
        f32x16_t acc[2][4];   // written from zero by the column block's first MFMAs
        const __amdgpu_buffer_rsrc_t prev = ui > 0 ? ys : ynull;  // unit 0 stores nothing, same count
        load_b(bf[0], g0, 0);
        load_b(bf[1], g0, 1);
#pragma unroll
        for (int kt = 0; kt < KTM; ++kt) {
            if (kt < KT) {
                const int g = g0 + kt;
#pragma unroll
                for (int s = 0; s < kSub; ++s) {
                    const int q = kt * kSub + s;                      // step within the column block
                    const bool next1 = s + 1 < kSub || kt + 1 < KT;   // step q+1 exists
                    const bool next2 = s + 2 < kSub || kt + 1 < KT;   // step q+2 exists
                    if (next1) wait_lgkm_n<kLoads>();
                    else wait_lgkm0();
                    if (s == kSub - 2 && g + 1 < nstages) stage_ready(g + 1, (kt + 1) % KTM);
                    const bool st = s == 0 && has_st(kt);
                    u32x4_t yv[kChunks];
                    if (st) read_y_chunks<kChunks>(stage, kChunks * kt, tid, yv);
                    if (next2) {
                        const int s2_ = (s + 2) % kSub;
                        load_b(bf[(q + 2) % 3], s + 2 < kSub ? g : g + 1, s2_);
                    }
                    APS_PIN();
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            // the folded kernels' register pressure puts B
                            // fragments in AGPRs, copied back right before use
                            if (q == 0) Fmt::template mma_pinned_first<FOLD != 0>(acc[i][j], bf[q % 3][j], areg[kt][i][s]);
                            else Fmt::template mma_pinned<FOLD != 0>(acc[i][j], bf[q % 3][j], areg[kt][i][s]);
                        }
                    APS_PIN();
                    if (st && (FOLD == 0 || ui > 0)) {
                        // the previous column block's chunks kChunks kt ..
                        if constexpr (FOLD == 0) {
                            write_y_chunks<4>(prev, H, nb - 1, 4 * kt, tid, yv);
                        } else {
#pragma unroll
                            for (int c = 0; c < kChunks; ++c)
                                __builtin_amdgcn_raw_buffer_store_b128(yv[c], ys,
                                                                       tok_off(rowoff[kChunks * kt + c], nb - 1, tid), 0, 0);
                        }
                        APS_PIN();
                    }
                    if constexpr (FOLD == 2) {
                        if (s == 0 && kt == 2) {
                            // every wave has read the stage out (the barrier of
                            // this step's stage_ready): this tile's ya rows go in
                            issue_ya(nb);
                            APS_PIN();
                        }
                    }
                }
            }
        }

        // epilogue: scales (fp8), bf16, staged in LDS
        if constexpr (Fmt::kPinned) asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");  // MFMA write -> VALU read
        if constexpr (FOLD == 2) {
            // this wave's ya copies have landed (issued at k stage 2; since:
            // the ring copies of k stage 3's stage_ready, if it ran one); the
            // barrier below makes every wave's visible
            const int g3 = g0 + 3;
            wait_vm_lgkm0_n(g3 + 1 < nstages && g3 + 3 < nstages ? 4 : 0);
        }
        if (kOverlap) raw_barrier();  // every thread has read the previous tile out of the stage
        // Column fragment by column fragment (32 columns, both row
        // fragments): its LDS reads (fp8 column scales, FOLD 2's slot-0
        // values) are issued before the previous fragment's stores, so that
        // waiting for them does not wait for those stores (LDS operations
        // complete in order: read, store, read, store would cost one LDS
        // round trip per four columns).
        float4 sc4[2][4];
        u32x2_t ya4[2][2][4];
        auto epi_reads = [&](int j, float4 (&sc)[4], u32x2_t (&ya)[2][4]) __attribute__((always_inline)) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int col = 32 * j + 8 * q + 4 * (lane >> 5);
                if constexpr (kFp8) sc[q] = *reinterpret_cast<const float4*>(lds.scl + ui * 128 + col);
                if constexpr (FOLD == 2) {
#pragma unroll
                    for (int i = 0; i < 2; ++i)
                        ya[i][q] = *reinterpret_cast<const u32x2_t*>(stage + (aR + i * 32 + (lane & 31)) * kArPitch + col);
                }
            }
        };
        epi_reads(0, sc4[0], ya4[0]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (j + 1 < 4) epi_reads(j + 1, sc4[(j + 1) & 1], ya4[(j + 1) & 1]);
            const float4 (&sc)[4] = sc4[j & 1];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = aR + i * 32 + (lane & 31);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float o[4];
#pragma unroll
                    for (int v = 0; v < 4; ++v) o[v] = acc[i][j][4 * q + v];
                    const int col = 32 * j + 8 * q + 4 * (lane >> 5);
                    if constexpr (kFp8) {
                        o[0] = o[0] * rs[i] * sc[q].x; o[1] = o[1] * rs[i] * sc[q].y;
                        o[2] = o[2] * rs[i] * sc[q].z; o[3] = o[3] * rs[i] * sc[q].w;
                    }
                    u32x2_t* at = reinterpret_cast<u32x2_t*>(stage + row * kArPitch + col);
                    const u32x2_t v = {pack2_bf16(o[0], o[1]), pack2_bf16(o[2], o[3])};
                    // FOLD 2: this row's slot-1 output (bf16, as y would hold
                    // it) combined with the token's slot-0 row in the stage
                    if constexpr (FOLD == 2) *at = combine4_bf16(ya4[j & 1][i][q], v);
                    else *at = v;
                }
            }
        }
        wait_lgkm0();
        raw_barrier();
        if constexpr (FOLD == 0) {
            if (!kOverlap || ui + 1 == nunits) {
                // no later column block to hide under: store the tile now
                u32x4_t yv[16];
                read_y_chunks<16>(stage, 0, tid, yv);
                write_y_chunks<16>(ys, H, nb, 0, tid, yv);
                if (!kOverlap) {
                    wait_lgkm0();
                    raw_barrier();  // the stage is read out before the next epilogue
                }
            }
        }
    }
    if constexpr (FOLD != 0) {
        // the last column block's tile, after the loop
        if (nunits > 0) {
            const int nb = u.nb1 - 1;
            u32x4_t yv[16];
            read_y_chunks<16>(stage, 0, tid, yv);
#pragma unroll
            for (int c = 0; c < 16; ++c)
                __builtin_amdgcn_raw_buffer_store_b128(yv[c], ys, tok_off(rowoff[c], nb, tid), 0, 0);
        }
    }
}


// The register-resident w2 kernel for KT k stages, or null when KT is past
// the register budget (the streamed kernel serves those shapes).
typedef void (*down_ar_fn)(const uint8_t*, int64_t, const uint32_t*, const uint8_t*, bf16_t*, int, int,
                           const float*, const float*, const uint32_t*, const uint32_t*, const uint32_t*, bf16_t*,
                           int64_t);
template <class Fmt>
down_ar_fn down_ar_kernel(int KT) {
    switch (KT) {
        case 1: return k_ffn_down_ar<Fmt, 1>;
        case 2: return k_ffn_down_ar<Fmt, 2>;
        case 3: return k_ffn_down_ar<Fmt, 3>;
        case 4: return k_ffn_down_ar<Fmt, 4>;
        case 5: return DownAr<Fmt>::kKtMax >= 5 ? k_ffn_down_ar<Fmt, (DownAr<Fmt>::kKtMax >= 5 ? 5 : 1)> : nullptr;
        case 6: return DownAr<Fmt>::kKtMax >= 6 ? k_ffn_down_ar<Fmt, (DownAr<Fmt>::kKtMax >= 6 ? 6 : 1)> : nullptr;
        case 7: return DownAr<Fmt>::kKtMax >= 7 ? k_ffn_down_ar<Fmt, (DownAr<Fmt>::kKtMax >= 7 ? 7 : 1)> : nullptr;
        default: return nullptr;
    }
}

// The folded combine's two passes for fp8's production k-stage count (KT =
// 4), or null.
down_ar_fn down_fold_kernel_fp8(int KT, int fold) {
    if (KT != 4) return nullptr;
    return fold == 1 ? k_ffn_down_ar<Fp8Fmt, 4, 1> : k_ffn_down_ar<Fp8Fmt, 4, 2>;
}

// Grid of the register-resident w2 kernel: about one block per CU, at least
// one per row tile, a multiple of the XCD count.
dim3 grid_ar(int64_t rows, int experts) {
    const int64_t tiles = max_row_tiles(2 * rows, kArRows, experts);
    const int64_t g = tiles > num_cus() ? tiles : num_cus();
    return dim3(static_cast<unsigned>(ceil_div(g, kXcds) * kXcds));
}

// Upper bound on the work-list length for A = 2 * rows positions.
int64_t max_blocks(int64_t rows, int nblk, int experts, bool all_tall) {
    if (all_tall) return max_row_tiles(2 * rows, 256, experts) * nblk;
    return max_row_tiles(2 * rows, 128, experts) * (nblk / 2) +
           ((nblk & 1) ? max_row_tiles(2 * rows, 256, experts) : 0);
}

dim3 grid_of(int64_t blocks) { return dim3(static_cast<unsigned>(ceil_div(blocks, kXcds) * kXcds)); }

// Persistent grid of the w1||w3 GEMM: one block per CU (a multiple of the
// XCD count); the kernel deals its pieces to them.
dim3 grid_up() {
    const int g = num_cus() / kXcds * kXcds;
    return dim3(static_cast<unsigned>(g > 0 ? g : kXcds));
}

}  // namespace

// Compute units of the current device (cached per device).
int num_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

hipError_t launch_ffn_up_bf16(const bf16_t* x, const uint32_t* offsets,
                              const uint32_t* assignment_rows, const bf16_t* w13,
                              bf16_t* act, int64_t rows, int hidden, int ffn, int experts,
                              hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hidden % 64 != 0 || ffn % 64 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_ffn_up<Bf16Fmt>, grid_up(), dim3(256), 0, s,
                       reinterpret_cast<const uint8_t*>(x), static_cast<int64_t>(hidden) * 2, offsets,
                       assignment_rows, reinterpret_cast<const uint8_t*>(w13), act, hidden, ffn, experts,
                       nullptr, nullptr, nullptr);
    return hipGetLastError();
}

hipError_t launch_ffn_down_bf16(const bf16_t* act, const uint32_t* offsets, const bf16_t* w2,
                                bf16_t* y, int64_t rows, int hidden, int ffn, int experts,
                                hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hidden % 128 != 0 || ffn % 64 != 0) return hipErrorInvalidValue;
    if (auto kern = down_ar_kernel<Bf16Fmt>(ffn / 64)) {
        hipLaunchKernelGGL(kern, grid_ar(rows, experts), dim3(256), 0, s,
                           reinterpret_cast<const uint8_t*>(act), static_cast<int64_t>(ffn) * 2, offsets,
                           reinterpret_cast<const uint8_t*>(w2), y, hidden, experts, nullptr, nullptr, nullptr,
                           nullptr, nullptr, nullptr, rows);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_ffn_down<Bf16Fmt>, grid_of(max_blocks(rows, hidden / 128, experts, APS_DOWN_TALL)),
                       dim3(256), 0, s, reinterpret_cast<const uint8_t*>(act), static_cast<int64_t>(ffn) * 2,
                       offsets, reinterpret_cast<const uint8_t*>(w2), y, hidden, ffn / 64, experts, nullptr,
                       nullptr);
    return hipGetLastError();
}

hipError_t launch_ffn_up_fp8(const uint8_t* xq, const float* x_scale, const uint32_t* offsets,
                             const uint32_t* assignment_rows, const uint8_t* w13, const float* w1_scale,
                             const float* w3_scale, bf16_t* act, int64_t rows, int hidden, int ffn,
                             int experts, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hidden % 128 != 0 || ffn % 64 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_ffn_up<Fp8Fmt>, grid_up(), dim3(256), 0, s,
                       xq, static_cast<int64_t>(hidden), offsets, assignment_rows, w13, act, hidden, ffn, experts,
                       x_scale, w1_scale, w3_scale);
    return hipGetLastError();
}

hipError_t launch_ffn_down_fp8(const uint8_t* actq, const float* act_scale, const uint32_t* offsets,
                               const uint8_t* w2, const float* w2_scale, bf16_t* y, int64_t rows, int hidden,
                               int ffn, int experts, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hidden % 128 != 0 || ffn % 64 != 0) return hipErrorInvalidValue;
    const int kpad = static_cast<int>(ceil_div(ffn, 128) * 128);
    if (auto kern = down_ar_kernel<Fp8Fmt>(kpad / 128)) {
        hipLaunchKernelGGL(kern, grid_ar(rows, experts), dim3(256), 0, s, actq,
                           static_cast<int64_t>(kpad), offsets, w2, y, hidden, experts, act_scale, w2_scale,
                           nullptr, nullptr, nullptr, nullptr, rows);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_ffn_down<Fp8Fmt>, grid_of(max_blocks(rows, hidden / 128, experts, APS_DOWN_TALL)),
                       dim3(256), 0, s, actq, static_cast<int64_t>(kpad), offsets, w2, y, hidden, kpad / 128,
                       experts, act_scale, w2_scale);
    return hipGetLastError();
}

bool ffn_down_fold_fits(int64_t rows, int hidden, int ffn) {
    // byte offsets into the [rows][hidden] bf16 arrays stay below 2^31
    const int64_t bytes = rows * static_cast<int64_t>(hidden) * 2;
    return rows > 0 && hidden % 128 == 0 && ffn % 64 == 0 && ceil_div(ffn, 128) == 4 &&
           bytes + (int64_t(1) << 20) < (int64_t(1) << 31);
}

hipError_t launch_ffn_down_fold_fp8(const uint8_t* actq, const float* act_scale, const uint32_t* offsets,
                                    const uint32_t* slot1, const uint32_t* slot_rows, const uint32_t* slot_tokens,
                                    const uint8_t* w2, const float* w2_scale, bf16_t* ya, bf16_t* out,
                                    int64_t rows, int hidden, int ffn, int experts, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (!ffn_down_fold_fits(rows, hidden, ffn)) return hipErrorInvalidValue;
    const int kpad = static_cast<int>(ceil_div(ffn, 128) * 128);
    for (int fold = 1; fold <= 2; ++fold) {
        down_ar_fn kern = down_fold_kernel_fp8(kpad / 128, fold);
        if (!kern) return hipErrorInvalidValue;
        hipLaunchKernelGGL(kern, grid_ar(rows, experts), dim3(256), 0, s, actq, static_cast<int64_t>(kpad), offsets,
                           w2, ya, hidden, experts, act_scale, w2_scale, slot1, slot_rows, slot_tokens, out, rows);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace aps
