// fp32 Linear on the matrix cores, bit for bit the reference's FMA chain.
//
// y[m][n] = (fp32 FMA chain over k ascending of x[m][k] w[n][k]) + bias[n]:
// the decoder's projections.  Reference: Linear::forward (src/layer.cu:30-42)
// -> matmul_transposed_bias_gpu (src/tensor.cu:3120-3143) ->
// k_matmul_transposed_8x8 (src/tensor.cu:715-800): one accumulator per output
// walked over k ascending, the bias added once in the epilogue.
//
// gfx950's K = 1 fp32 MFMA, v_mfma_f32_32x32x1_2b_f32, computes D = A B + C
// for two 32 x 32 blocks with ONE fused multiply-add per element, so a chain
// of them over k ascending is the fmaf chain itself.  Measured on gfx950 over
// 4096-step chains (operands uniform, with exponents spread over 2^-20 ..
// 2^20, and with products around FLT_MIN): every output equal to the fused
// chain, none to the unfused one.  The projections thus run at the matrix
// cores' fp32 rate (256 FLOP per clock per CU) instead of the vector FMA
// rate (128 without packed math), with the same bits.
//
// Mapping.  A block computes 128 rows x 128 columns with four waves of
// 64 x 64 (64 columns with waves of 64 x 32 when the grid is small); a wave
// issues two MFMAs per k (columns 32j .. 32j+31, j = 0, 1):
// block 0 of an MFMA is rows 0..31 of the wave tile (A from lanes 0..31),
// block 1 rows 32..63 (lanes 32..63), both against the same 32 columns (B
// read twice).  Stages are 32 k deep: 128 x rows and 128 (64) weight rows
// of 128 bytes (32 KB), copied with global_load_lds_dwordx4 into two LDS slots;
// 16-byte chunks are XOR-swizzled by row pair, so the 16 lanes of an operand
// read (16 consecutive rows, one chunk) hit 16 distinct bank groups.  A lane
// reads four k of its row at once (one ds_read_b128) and feeds four MFMAs.
// Per CU the copy traffic is 8 bytes per 256 FLOP: the kernel is bound by
// the MFMA rate, not by loads.
#include "common.hpp"

#include <utility>

namespace aps {
namespace {

typedef float lf32x32_t __attribute__((ext_vector_type(32)));
typedef float lf32x4_t __attribute__((ext_vector_type(4)));

constexpr int kLRows = 128;               // x rows per block
constexpr int kLStageK = 32;              // k per stage: one 128-byte row

#define APS_LGP(p) ((const __attribute__((address_space(1))) void*)(p))
#define APS_LLP(p) ((__attribute__((address_space(3))) void*)(p))

__device__ inline int lswz(int row, int chunk) { return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4); }

template <int N>
__device__ inline void l_wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}
__device__ inline void l_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <int V>
struct LInt {
    static constexpr int value = V;
};

constexpr int kLXcds = 8;   // XCDs of an MI355X

// Up to three outputs of one x in one grid (the reference's
// matmul_pair_bias_gpu pairs k and v): segment s owns column tiles
// t0[s] .. t0[s + 1] - 1 of the grid's x dimension.
struct LinSegs {
    const float* w[3];
    const float* b[3];
    float* y[3];
    int n[3];
    int t0[4];
};

// WN: columns per wave (64: two MFMAs per k; 32: one, for grids that would
// otherwise leave CUs idle).  A block is 128 rows x 2 WN columns.
// The grid is one-dimensional over the row-tile-major tile order.
// Workgroups are dealt to the 8 XCDs round robin (workgroup b runs on XCD
// b % 8).  Taken in launch order (tile b), XCD x holds the column tiles
// c = x mod 8 of every row tile: it reads an eighth of W and all of x.  With
// xcd_rows, workgroup b takes tile (b % 8) * per + b / 8 instead: XCD x holds
// a contiguous run of tiles, the column tiles of a row tile sharing its x
// rows in one L2, and reads about an eighth of x and all of W.  The
// launcher picks xcd_rows when x is the larger operand by 3x or more.
template <int WN>
__global__ void __launch_bounds__(256, 2)
k_linear_mfma(const float* __restrict__ x, const LinSegs segs, int64_t M, int K, int row_tiles, int xcd_rows) {
    constexpr int kBRows = 2 * WN;                        // weight rows per block
    constexpr int kStageRows = kLRows + kBRows;
    constexpr int kLStageBytes = kStageRows * 128;
    constexpr int kSlots = kStageRows / 32;               // copies per wave per stage
    constexpr int NJ = WN / 32;                           // MFMAs per k
    // one LDS object for both slots: with two, the compiler's tracking of the
    // in-flight copies made every stage's first read wait for all of them
    // (the next stage's included); the waits here are explicit
    __shared__ __align__(16) uint8_t ring[2][kLStageBytes];
    uint8_t* const slot0 = ring[0];
    uint8_t* const slot1 = ring[1];
    const int ncol = segs.t0[3];
    const int64_t per = (static_cast<int64_t>(row_tiles) * ncol + kLXcds - 1) / kLXcds;
    const int64_t t = xcd_rows ? static_cast<int64_t>(blockIdx.x % kLXcds) * per + blockIdx.x / kLXcds
                               : static_cast<int64_t>(blockIdx.x);
    if (t >= static_cast<int64_t>(row_tiles) * ncol) return;
    const int tc = static_cast<int>(t % ncol);
    const int64_t m0 = (t / ncol) * kLRows;
    const int sg = tc >= segs.t0[1] ? (tc >= segs.t0[2] ? 2 : 1) : 0;
    const float* __restrict__ w = segs.w[sg];
    const float* __restrict__ bias = segs.b[sg];
    float* __restrict__ y = segs.y[sg];
    const int N = segs.n[sg];
    const int n0 = (tc - segs.t0[sg]) * kBRows;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int KT = K / kLStageK;

    // copies: instruction s of wave w fills stage rows 32s + 8w .. +7; lane
    // i writes row 32s + 8w + i/8, physical chunk i & 7, i.e. logical chunk
    // (i & 7) ^ ((row >> 1) & 7).  Rows 0..127 are x rows m0.., the rest
    // weight rows n0..; rows past the end re-read the last one (their
    // results are not stored).
    const float* src[kSlots];
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
        const int row = 32 * s + 8 * wave + (lane >> 3);
        const int chunk = (lane & 7) ^ ((row >> 1) & 7);
        if (row < kLRows) {
            const int64_t r = m0 + row < M ? m0 + row : M - 1;
            src[s] = x + r * K + 4 * chunk;
        } else {
            const int64_t r = n0 + (row - kLRows) < N ? n0 + (row - kLRows) : N - 1;
            src[s] = w + r * K + 4 * chunk;
        }
    }
    auto issue = [&](uint8_t* slot, int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < kSlots; ++s)
            __builtin_amdgcn_global_load_lds(APS_LGP(src[s] + kt * kLStageK),
                                             APS_LLP(slot + (32 * s + 8 * wave) * 128), 16, 0, 0);
    };

    const int aR = (wave & 1) * 64;            // this wave's x rows in the stage
    const int bR = kLRows + (wave >> 1) * WN;  // its weight rows
    lf32x32_t acc[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int v = 0; v < 32; ++v) acc[j][v] = 0.0f;

    // one stage: 8 groups of 4 k; the group's operands are read one group
    // ahead of its MFMAs
    auto compute = [&](const uint8_t* st) __attribute__((always_inline)) {
        lf32x4_t a[2], b[2][NJ];
        auto load = [&](int q, int p) __attribute__((always_inline)) {
            a[p] = *reinterpret_cast<const lf32x4_t*>(st + lswz(aR + lane, q));
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                b[p][j] = *reinterpret_cast<const lf32x4_t*>(st + lswz(bR + 32 * j + (lane & 31), q));
        };
        load(0, 0);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            if (q + 1 < 8) load(q + 1, (q + 1) & 1);
            const int p = q & 1;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    acc[j] = __builtin_amdgcn_mfma_f32_32x32x1f32(a[p][kk], b[p][j][kk], acc[j], 0, 0, 0);
        }
    };

    // double buffer: stage kt in slot kt % 2; after its MFMAs and a barrier
    // the slot takes stage kt + 2
    auto run = [&](auto par, int kt) __attribute__((always_inline)) {
        constexpr int P = decltype(par)::value;
        uint8_t* slot = P ? slot1 : slot0;
        if (kt + 1 < KT) l_wait_vm<kSlots>();
        else l_wait_vm<0>();
        l_barrier();
        compute(slot);
        l_barrier();
        if (kt + 2 < KT) issue(slot, kt + 2);
    };
    issue(slot0, 0);
    if (KT > 1) issue(slot1, 1);
    for (int kt = 0; kt < KT; kt += 2) {
        run(LInt<0>{}, kt);
        if (kt + 1 < KT) run(LInt<1>{}, kt + 1);
    }

    // epilogue: register v of acc[j] is row 32 (v / 16) + 8 ((v % 16) / 4)
    // + 4 (lane / 32) + v % 4 of the wave tile, column 32 j + lane % 32; the
    // 32 lanes of a row store 128 contiguous bytes
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int col = n0 + (wave >> 1) * WN + 32 * j + (lane & 31);
        const bool col_ok = col < N;
        const float bb = (bias != nullptr && col_ok) ? bias[col] : 0.0f;
#pragma unroll
        for (int v = 0; v < 32; ++v) {
            const int64_t row = m0 + aR + 32 * (v / 16) + 8 * ((v % 16) / 4) + 4 * (lane >> 5) + (v % 4);
            if (row < M && col_ok) y[row * N + col] = bias != nullptr ? __fadd_rn(acc[j][v], bb) : acc[j][v];
        }
    }
}

}  // namespace

bool linear_mfma_fits(int64_t rows, int in_f, int out_f) {
    return rows > 0 && in_f > 0 && in_f % kLStageK == 0 && out_f > 0 && (rows + kLRows - 1) / kLRows <= 65535;
}

hipError_t launch_linear_mfma_multi(const float* x, int64_t rows, int in_f, int count, const float* const* w,
                                    const float* const* bias, float* const* y, const int* out_f, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (count < 1 || count > 3) return hipErrorInvalidValue;
    for (int i = 0; i < count; ++i)
        if (!linear_mfma_fits(rows, in_f, out_f[i])) return hipErrorInvalidValue;
    // 128- or 64-column blocks, whichever gives the busiest CU less work:
    // blocks per CU (rounded up) x width, the 64-column block charged 5% for
    // its lower FLOP rate and either charged 30% when the grid leaves CUs
    // fewer than two workgroups (no latency hiding between them)
    const int64_t cus = num_cus(), rt = ceil_div(rows, kLRows);
    auto cost = [&](int bc, double rate) {
        int64_t tiles = 0;
        for (int i = 0; i < count; ++i) tiles += ceil_div(out_f[i], bc) * rt;
        return static_cast<double>(ceil_div(tiles, cus) * bc) * rate * (tiles < 2 * cus ? 1.3 : 1.0);
    };
    const bool wide = cost(128, 1.0) <= cost(64, 1.05);
    const int bc = wide ? 128 : 64;
    LinSegs segs{};
    int t = 0;
    for (int i = 0; i < 3; ++i) {
        segs.t0[i] = t;
        if (i < count) {
            segs.w[i] = w[i];
            segs.b[i] = bias[i];
            segs.y[i] = y[i];
            segs.n[i] = out_f[i];
            t += static_cast<int>(ceil_div(out_f[i], bc));
        }
    }
    segs.t0[3] = t;
    for (int i = count; i < 3; ++i) segs.t0[i] = t;   // empty segments past the last
    const int64_t tiles = static_cast<int64_t>(t) * rt;
    int64_t wcols = 0;
    for (int i = 0; i < count; ++i) wcols += out_f[i];
    const int xr = rows >= 3 * wcols ? 1 : 0;   // x bytes >= 3 x W bytes (both rows x in_f fp32)
    const dim3 grid(static_cast<unsigned>(ceil_div(tiles, kLXcds) * kLXcds));
    if (wide) hipLaunchKernelGGL(k_linear_mfma<64>, grid, dim3(256), 0, s, x, segs, rows, in_f, static_cast<int>(rt), xr);
    else hipLaunchKernelGGL(k_linear_mfma<32>, grid, dim3(256), 0, s, x, segs, rows, in_f, static_cast<int>(rt), xr);
    return hipGetLastError();
}

hipError_t launch_linear_mfma_f32(const float* x, const float* w, const float* bias, float* y, int64_t rows,
                                  int in_f, int out_f, hipStream_t s) {
    return launch_linear_mfma_multi(x, rows, in_f, 1, &w, &bias, &y, &out_f, s);
}

}  // namespace aps
