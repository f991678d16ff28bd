// Rotary embedding and GQA tree attention over the prefix-trie rows.
//
// Reference: k_rope (src/tensor.cu:2180-2197) behind apply_rope_tree_gpu
// (src/tensor.cu:3342-3359), and k_attention_tree_gqa4 (src/tensor.cu:
// 2407-2633) behind attention_tree_gpu (src/tensor.cu:3361-3377).  A row is
// a trie node: its RoPE position is its depth and its keys are its ancestor
// chain (the last SLIDING_WINDOW of it), so attention runs on deduplicated
// rows without expanding them back to tokens.
//
// Arithmetic kept from the reference kernel, operation for operation, so the
// result is the reference's to the bit (up to the double exp below):
//   score of key w for query head g:
//     a_j = fma chain over d = j, j + 4, ... ascending (j < 4), +0 init
//     s_w = ((a_0 + a_1) + (a_2 + a_3)) * (1 / sqrtf(head_dim))
//   m = max_w s_w;  e_w = (float)exp((double)(s_w - m));
//   den = fp32 sum of e_w over w ascending (one lane per head);  p_w = e_w / den
//   out[d] = fma chain over w ascending of p_w * v[key w][d]
// exp is ROCm's double exp (the reference: CUDA's); both are within an ulp of
// double, so the float e_w agree except when a double lands within an ulp of
// a float rounding boundary.
//
// gfx950 mapping.  Path groups (4 consecutive rows on one ancestor chain,
// the common case) go to k_attention_group on the matrix cores (its own
// comment has the mapping); k_attention_tree serves the other rows: one
// 256-thread workgroup per (row, KV head) serves the four query heads of the
// group, as in the reference.  Scores: a thread owns a key and reads its
// 128-float row as 16-byte vectors, one element per partial sum a_0..a_3
// (the four partials are exactly the four lanes of a float4), against the
// four query rows broadcast from LDS.  The order-critical denominator runs
// on four lanes (one per head) of one wave.  Values: a thread owns one
// dimension d of two heads and walks the keys in order, V rows read
// coalesced (128 threads = one 512-byte row).
#include "common.hpp"

namespace aps {
namespace {

constexpr int kHeadDim = 128;
constexpr int kGroup = 4;            // query heads per KV head (GQA-4)
constexpr int kAttnThreads = 256;

typedef float af4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256)
k_rope_tree(float* __restrict__ x, const uint32_t* __restrict__ row_pos, int64_t rows, int heads, int half,
            const float* __restrict__ cosv, const float* __restrict__ sinv, int64_t max_seq) {
    const int64_t pair = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (pair >= rows * heads * half) return;
    const int j = static_cast<int>(pair % half);
    const int64_t rh = pair / half;  // row * heads + head
    const int64_t row = rh / heads;
    const uint32_t pos = row_pos[row];
    if (pos >= max_seq) return;  // outside the table: left as is (the C++ layer checks positions)
    float* base = x + rh * (2 * half);
    const int64_t t = static_cast<int64_t>(pos) * half + j;
    const float c = cosv[t], s = sinv[t];
    const float x0 = base[j], x1 = base[j + half];
    base[j] = __fmaf_rn(x0, c, -__fmul_rn(x1, s));
    base[j + half] = __fmaf_rn(x1, c, __fmul_rn(x0, s));
}

// ---------------------------------------------------------------------------
// Row groups on the matrix cores.  Rows are taken 4 at a time (group g =
// rows 4g .. 4g+3).  A group is a path group when every row lies on the
// ancestor chain of the group's last row (tree: anc[last][pos[r]] == r;
// packed: one sequence), so each row's keys are a contiguous range of that
// one chain.  k_attention_group serves path groups; the row kernel below the
// others.  Both evaluate this predicate the same way, on the same clamped
// positions.
constexpr int kGroupRows = 4;
constexpr int kGroupQueries = kGroupRows * kGroup;   // 16: query q = 4 row + head
constexpr int kKeyTile = 16;                         // keys per score tile / value group

template <bool PACKED>
__device__ inline bool group_is_path(const uint32_t* __restrict__ row_pos, const uint32_t* __restrict__ anc,
                                     int64_t anc_stride, int64_t rows, int64_t r0, int wmax, int cap, int lane) {
    const int nr = static_cast<int>(rows - r0 < kGroupRows ? rows - r0 : kGroupRows);
    const int64_t last = r0 + nr - 1;
    bool ok = true;
    int64_t pr = 0;
    if (lane < nr) {
        const int64_t r = r0 + lane;
        pr = row_pos[r];
        pr = pr < anc_stride ? pr : anc_stride - 1;
        if (PACKED) ok = anc[r] == anc[last];
        else ok = anc[last * anc_stride + pr] == static_cast<uint32_t>(r);
    }
    // the group's key range chain[dlo .. plast] must hold every row's window
    // and fit the kernel's LDS (cap keys)
    const int64_t p0 = __shfl(pr, 0), plast = __shfl(pr, nr - 1);
    if (lane < nr) ok = ok && pr >= p0 && pr <= plast;
    const int64_t dlo = p0 + 1 > wmax ? p0 + 1 - wmax : 0;
    return __all(ok) && plast - dlo + 1 <= cap;
}

typedef float ag16_t __attribute__((ext_vector_type(16)));

// 4 x 4 transpose across the four 16-lane rows of a wave: on entry row R
// holds x[c] = element 4 R + c of a 16-element run; on exit row R holds
// x[r] = element 4 r + R.  Two v_permlane32_swap (rows 2, 3 of the first
// operand <-> rows 0, 1 of the second) and two v_permlane16_swap (odd rows of
// the first <-> even rows of the second).
__device__ inline void rows_transpose4(af4& x) {
    // (__float_as_uint on the element values: a bit cast of an element
    // lvalue of a vector reads element 0)
    const uint32_t a = __float_as_uint(x[0]), b = __float_as_uint(x[1]);
    const uint32_t c = __float_as_uint(x[2]), d = __float_as_uint(x[3]);
    auto ac = __builtin_amdgcn_permlane32_swap(a, c, false, false);
    auto bd = __builtin_amdgcn_permlane32_swap(b, d, false, false);
    auto ab = __builtin_amdgcn_permlane16_swap(ac[0], bd[0], false, false);
    auto cd = __builtin_amdgcn_permlane16_swap(ac[1], bd[1], false, false);
    x[0] = __uint_as_float(ab[0]);
    x[1] = __uint_as_float(ab[1]);
    x[2] = __uint_as_float(cd[0]);
    x[3] = __uint_as_float(cd[1]);
}

// One workgroup = one path group x one KV head: 16 queries (4 rows x the
// group's 4 query heads) against the keys chain[dlo .. dhi] of the group's
// last row; row r attends to chain[begin_r .. pos_r].  The arithmetic is the
// row kernel's, operation for operation:
//   scores on the K = 1 fp32 MFMA v_mfma_f32_16x16x1_4b_f32 (one fused
//     multiply-add per element and step, the fmaf chain): its four blocks are
//     the four partial chains a_j over d = j, j + 4, .. (block j: A = q[d],
//     B = k[d] with d = 4 i + j at step i), for 16 queries x 16 keys; then
//     s = ((a0 + a1) + (a2 + a3)) * scale in registers, into LDS;
//   per query over its window: m = max s, e = (float)exp((double)(s - m)),
//     den = sum of e in key order (one lane per query), p = e / den;
//   out[d] = chain over keys of p v[d] on the same MFMA: blocks are four
//     16-dimension groups, A = p (lane = query), B = v.
// Every score is computed once: the group's 16 x window scores sit in LDS.
// Keys after a row's window take p = 0, which leaves its value chains
// unchanged except that a -0 would turn +0; keys before it keep the chain
// at its +0 start.
//   K and V go from global memory straight to registers (LDS holds only the
// scores and the chain's key rows, so two workgroups fit a CU at 1,024-key
// windows, and three, MINB = 3 with 168 registers, at key spans up to 784).  Scores: wave w takes the 16-key tiles w, w + 4, ..; a lane
// (key lane % 16, row j = lane / 16) loads 16 bytes of elements 16 a + 4 j ..
// per a < 8 and a 4 x 4 transpose across the rows gives it d = 4 i + j,
// tiles two ahead in flight.  Softmax: the 16 threads of query q are in
// wave q / 4, so exp, the ordered denominator and p = e / den need no
// workgroup barrier.  Values: two waves (0, 1 on even workgroups, 2, 3 on
// odd ones, so that two resident workgroups spread them over the SIMDs) take
// dimensions 64 w' .. 64 w' + 63, one coalesced 256-byte load per key, 64
// keys ahead; the K / V row offsets are 32-bit byte offsets off a uniform
// base.
template <bool PACKED, int MINB>
__global__ void __launch_bounds__(256, MINB)
k_attention_group(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
                  float* __restrict__ out, const uint32_t* __restrict__ row_pos, const uint32_t* __restrict__ anc,
                  int64_t anc_stride, int64_t rows, int q_heads, int kv_heads, int wmax, float scale, int sw) {
    extern __shared__ __align__(16) float gdyn[];
    float* sc = gdyn;                                                     // [16 queries][sw]: s, then e
    uint32_t* chain = reinterpret_cast<uint32_t*>(sc + kGroupQueries * sw);   // [sw - 1] key rows
    __shared__ int qlo[kGroupQueries], qhi[kGroupQueries];   // window of each query, relative to dlo
    __shared__ float wmx[4][kGroupQueries];                  // per-wave maxima

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // groups in reverse row order: later rows (longer chains in trie and
    // packed order) start first, so the short ones fill the last round
    const int64_t r0 = static_cast<int64_t>(gridDim.x / kv_heads - 1 - blockIdx.x / kv_heads) * kGroupRows;
    const int kh = static_cast<int>(blockIdx.x % kv_heads);
    // sw = key capacity + 1; groups that are not path groups are the row kernel's
    if (!group_is_path<PACKED>(row_pos, anc, anc_stride, rows, r0, wmax, sw - 1, lane)) return;
    const int nr = static_cast<int>(rows - r0 < kGroupRows ? rows - r0 : kGroupRows);
    const int64_t last = r0 + nr - 1;
    auto pos_of = [&](int64_t r) -> int64_t {
        const int64_t p = row_pos[r];
        return p < anc_stride ? p : anc_stride - 1;
    };
    const int64_t plast = pos_of(last);
    const int64_t p0 = pos_of(r0);
    const int dlo = static_cast<int>(p0 + 1 > wmax ? p0 + 1 - wmax : 0);
    const int dhi = static_cast<int>(plast);
    const int W = dhi - dlo + 1;
    const int ntiles = (W + kKeyTile - 1) / kKeyTile;   // 16-key tiles (at most capacity / 16)
    const int64_t seg = PACKED ? static_cast<int64_t>(anc[last]) : 0;
    if (tid < kGroupQueries) {
        const int r = tid / kGroup;
        if (r < nr) {
            const int64_t pr = pos_of(r0 + r);
            qhi[tid] = static_cast<int>(pr) - dlo;
            qlo[tid] = static_cast<int>(pr + 1 > wmax ? pr + 1 - wmax : 0) - dlo;
        } else {
            qhi[tid] = -1;   // a padding row: an empty window
            qlo[tid] = 0;
        }
    }
    // q operand: lane l -> query l % 16 (row (l % 16) / 4, head (l % 16) % 4),
    // element d = 4 i + l / 16 at step i (loads in flight during the staging)
    const int qq = lane & 15, qj = lane >> 4;
    const int qrow = qq / kGroup;
    const int64_t qr = r0 + (qrow < nr ? qrow : nr - 1);
    const float* qsrc = q + (qr * q_heads + kh * kGroup + qq % kGroup) * kHeadDim + qj;
    float qv[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) qv[i] = qsrc[4 * i];
    // the chain's key rows (clamped to the chain and the rows) in LDS, as
    // byte offsets of the key's K / V row (below 2^32: the launcher's check)
    const uint32_t kvs_bytes = static_cast<uint32_t>(kv_heads) * kHeadDim * sizeof(float);
    for (int i = tid; i < ntiles * 16; i += 256) {
        const int d = dlo + i < dhi ? dlo + i : dhi;
        const int64_t a = PACKED ? seg + d : static_cast<int64_t>(anc[last * anc_stride + d]);
        chain[i] = static_cast<uint32_t>(a < rows ? a : rows - 1) * kvs_bytes;
    }
    __syncthreads();
    // this lane's four score queries 4 qj + t: windows
    int lo[4], hi[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        lo[t] = qlo[4 * qj + t];
        hi[t] = qhi[4 * qj + t];
    }

    // ---- scores: tiles wave, wave + 4, .. ----
    const char* const kbase = reinterpret_cast<const char*>(k + kh * kHeadDim);
    auto kload = [&](int t, af4* buf) __attribute__((always_inline)) {
        const af4* src = reinterpret_cast<const af4*>(kbase + (chain[16 * t + qq] + 16u * qj));
#pragma unroll
        for (int a = 0; a < 8; ++a) buf[a] = src[4 * a];
    };
    float m[4] = {-3.402823466e+38f, -3.402823466e+38f, -3.402823466e+38f, -3.402823466e+38f};
    // the loads of every step are unconditional (a step past the end reloads
    // the last tile): the compiler's wait counts then leave the other
    // buffer's loads in flight
    auto tclamp = [&](int t) { return t < ntiles ? t : ntiles - 1; };
    auto tile = [&](int t, af4* buf) __attribute__((always_inline)) {
        float kvv[32];
#pragma unroll
        for (int a = 0; a < 8; ++a) {
            af4 x = buf[a];
            rows_transpose4(x);
#pragma unroll
            for (int r = 0; r < 4; ++r) kvv[4 * a + r] = x[r];
        }
        kload(tclamp(t + 8), buf);   // this wave's tile two ahead into the freed registers
        if (t >= ntiles) return;     // wave-uniform
        ag16_t acc = {};
#pragma unroll
        for (int i = 0; i < 32; ++i) acc = __builtin_amdgcn_mfma_f32_16x16x1f32(qv[i], kvv[i], acc, 0, 0, 0);
        // register 4 j + u: partial j of query 4 qj + u, key lane % 16
        const int w = 16 * t + qq;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float sx = __fmul_rn(__fadd_rn(__fadd_rn(acc[u], acc[4 + u]), __fadd_rn(acc[8 + u], acc[12 + u])),
                                       scale);
            sc[(4 * qj + u) * sw + w] = sx;
            if (w >= lo[u] && w <= hi[u]) m[u] = fmaxf(m[u], sx);
        }
    };
    if (wave < ntiles) {
        af4 kb0[8], kb1[8];
        kload(wave, kb0);
        kload(tclamp(wave + 4), kb1);
        for (int t = wave; t < ntiles; t += 8) {
            tile(t, kb0);
            tile(t + 4, kb1);
        }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) m[u] = fmaxf(m[u], __shfl_xor(m[u], o));
        if (qq == 0) wmx[wave][4 * qj + u] = m[u];
    }
    __syncthreads();

    // ---- softmax, per query on the 16 threads of one wave (queries
    // 4 w .. 4 w + 3 on wave w), so it needs no workgroup barrier ----
    const int qi = tid / 16, part = tid % 16;
    const int pw0 = 2 * (blockIdx.x & 1);             // waves pw0, pw0 + 1 take the values
    const int pwave = wave - pw0;                     // 0, 1 on those waves
    const int dim = 64 * pwave + 16 * qj + qq;        // their B column
    const char* const vbase = reinterpret_cast<const char*>(v + kh * kHeadDim);   // uniform: 32-bit lane offsets
    const uint32_t dbytes = static_cast<uint32_t>(dim) * sizeof(float);
    auto vload = [&](int g, float* vb) __attribute__((always_inline)) {
        const uint4* cr = reinterpret_cast<const uint4*>(chain + 16 * g);
#pragma unroll
        for (int u4 = 0; u4 < 4; ++u4) {
            const uint4 kr = cr[u4];
            vb[4 * u4 + 0] = *reinterpret_cast<const float*>(vbase + (kr.x + dbytes));
            vb[4 * u4 + 1] = *reinterpret_cast<const float*>(vbase + (kr.y + dbytes));
            vb[4 * u4 + 2] = *reinterpret_cast<const float*>(vbase + (kr.z + dbytes));
            vb[4 * u4 + 3] = *reinterpret_cast<const float*>(vbase + (kr.w + dbytes));
        }
    };
    float vb0[16], vb1[16], vb2[16], vb3[16];
    auto gclamp = [&](int g) { return g < ntiles ? g : ntiles - 1; };
    if (pwave == 0 || pwave == 1) {   // the first 64 keys' values go out now
        vload(0, vb0);
        vload(gclamp(1), vb1);
        vload(gclamp(2), vb2);
        vload(gclamp(3), vb3);
    }
    {
        const float mq = fmaxf(fmaxf(wmx[0][qi], wmx[1][qi]), fmaxf(wmx[2][qi], wmx[3][qi]));
        float* const srow = sc + qi * sw;
        const int l0 = qlo[qi], h0 = qhi[qi];
        // e = (float)exp((double)(s - m)) over the window, in place
        int w = l0 + part;
        for (; w + 48 <= h0; w += 64) {
            float x[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) x[u] = srow[w + 16 * u];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                srow[w + 16 * u] = static_cast<float>(exp(static_cast<double>(__fsub_rn(x[u], mq))));
        }
        for (; w <= h0; w += 16) srow[w] = static_cast<float>(exp(static_cast<double>(__fsub_rn(srow[w], mq))));
        // the denominator in key order on the query's first lane (the
        // wave's LDS accesses complete in program order), 16 reads ahead;
        // the wave barrier keeps the compiler from moving the other lanes'
        // stores past that lane's reads (they communicate through LDS)
        __builtin_amdgcn_wave_barrier();
        float den = 0.0f;
        if (part == 0) {
            int x = l0;
            for (; x + 16 <= h0 + 1; x += 16) {
                float e[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) e[u] = srow[x + u];
#pragma unroll
                for (int u = 0; u < 16; ++u) den = __fadd_rn(den, e[u]);
            }
            for (; x <= h0; ++x) den = __fadd_rn(den, srow[x]);
        }
        den = __shfl(den, lane & ~15);
        // p = e / den in the window, 0 elsewhere over the tiles
        int x = part;
        for (; x + 48 < ntiles * kKeyTile; x += 64) {
            float e[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) e[u] = srow[x + 16 * u];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int xu = x + 16 * u;
                srow[xu] = (xu >= l0 && xu <= h0) ? __fdiv_rn(e[u], den) : 0.0f;
            }
        }
        for (; x < ntiles * kKeyTile; x += 16) srow[x] = (x >= l0 && x <= h0) ? __fdiv_rn(srow[x], den) : 0.0f;
    }
    __syncthreads();

    // ---- values: out[q][d] = chain over keys of p v[d] (waves pw0, pw0 + 1) ----
    if (pwave != 0 && pwave != 1) return;
    ag16_t o = {};   // register 4 j + t: dimension 64 pwave + 16 j + lane % 16, query 4 (lane / 16) + t
    {
        const float* prow = sc + qq * sw;                   // A: query lane % 16
        auto group = [&](int g, float* vb) __attribute__((always_inline)) {
            float vc[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) vc[u] = vb[u];
            vload(gclamp(g + 4), vb);   // unconditional, as for the scores
            if (g >= ntiles) return;                           // wave-uniform
            float pa[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) pa[u] = prow[16 * g + u];
#pragma unroll
            for (int u = 0; u < 16; ++u) o = __builtin_amdgcn_mfma_f32_16x16x1f32(pa[u], vc[u], o, 0, 0, 0);
        };
        for (int g = 0; g < ntiles; g += 4) {
            group(g, vb0);
            group(g + 1, vb1);
            group(g + 2, vb2);
            group(g + 3, vb3);
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int qx = 4 * qj + t;                      // query: row qx / 4, head qx % 4
            const int r = qx / kGroup;
            if (r < nr)
                out[((r0 + r) * q_heads + kh * kGroup + qx % kGroup) * kHeadDim + 64 * pwave + 16 * j + qq] =
                    o[4 * j + t];
        }
}

// Dynamic LDS: scores [wmax][4] fp32, then chain [wmax] u32.
// PACKED: the rows are packed token sequences (reference k_attention_grouped_gqa4,
// src/tensor.cu:2267-2405, which the tree kernel restates with an index
// indirection): `anc` holds each row's segment start seg_offset[row], the
// keys of a row are the contiguous rows seg_offset + begin .. seg_offset +
// pos, and anc_stride is the longest segment.  Otherwise the keys are the
// ancestor chain anc[row][begin .. pos] of a trie node.
template <bool PACKED>
__global__ void __launch_bounds__(kAttnThreads)
k_attention_tree(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
                 float* __restrict__ out, const uint32_t* __restrict__ row_pos, const uint32_t* __restrict__ anc,
                 int64_t anc_stride, int64_t rows, int q_heads, int kv_heads, int wmax, float scale,
                 int group_cap) {
    extern __shared__ __align__(16) float dyn[];
    float* sc = dyn;                                                  // [w][g]
    uint32_t* chain = reinterpret_cast<uint32_t*>(dyn + static_cast<int64_t>(wmax) * kGroup);
    __shared__ __align__(16) float qs[kHeadDim][kGroup];              // [d][g]
    __shared__ float red[kAttnThreads / kWave][kGroup];
    __shared__ float stat[2][kGroup];                                 // max, denominator
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t row = blockIdx.x / kv_heads;
    const int kh = static_cast<int>(blockIdx.x % kv_heads);
    if (group_cap > 0 &&
        group_is_path<PACKED>(row_pos, anc, anc_stride, rows, row / kGroupRows * kGroupRows, wmax, group_cap, lane))
        return;  // k_attention_group's row
    // Positions past the ancestor table and key rows past the end are
    // clamped, for memory safety only: the C++ layer checks them (through
    // RowIndexBuffer::max_row and the packed segment table), and direct
    // C-ABI callers must keep them in range.
    int64_t pos = row_pos[row];
    pos = pos < anc_stride ? pos : anc_stride - 1;
    const int64_t begin = pos + 1 > wmax ? pos + 1 - wmax : 0;
    const int window = static_cast<int>(pos - begin + 1);
    const int64_t seg = PACKED ? static_cast<int64_t>(anc[row]) : 0;
    for (int i = tid; i < window; i += kAttnThreads) {
        const int64_t a = PACKED ? seg + begin + i : static_cast<int64_t>(anc[row * anc_stride + begin + i]);
        chain[i] = static_cast<uint32_t>(a < rows ? a : rows - 1);
    }
    for (int i = tid; i < kGroup * kHeadDim; i += kAttnThreads) {
        const int g = i / kHeadDim, d = i % kHeadDim;
        qs[d][g] = q[(row * q_heads + kh * kGroup + g) * kHeadDim + d];
    }
    __syncthreads();

    // ---- scores and the per-head maximum ----
    float mx[kGroup];
#pragma unroll
    for (int g = 0; g < kGroup; ++g) mx[g] = -3.402823466e+38f;
    for (int w = tid; w < window; w += kAttnThreads) {
        const af4* kr = reinterpret_cast<const af4*>(k + (static_cast<int64_t>(chain[w]) * kv_heads + kh) * kHeadDim);
        float a[kGroup][4];
#pragma unroll
        for (int g = 0; g < kGroup; ++g) a[g][0] = a[g][1] = a[g][2] = a[g][3] = 0.0f;
#pragma unroll 4
        for (int i = 0; i < kHeadDim / 4; ++i) {
            const af4 kv = kr[i];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const af4 qv = *reinterpret_cast<const af4*>(&qs[4 * i + j][0]);  // the four heads at d = 4i + j
                a[0][j] = __fmaf_rn(qv[0], kv[j], a[0][j]);
                a[1][j] = __fmaf_rn(qv[1], kv[j], a[1][j]);
                a[2][j] = __fmaf_rn(qv[2], kv[j], a[2][j]);
                a[3][j] = __fmaf_rn(qv[3], kv[j], a[3][j]);
            }
        }
        af4 s;
#pragma unroll
        for (int g = 0; g < kGroup; ++g) {
            s[g] = __fmul_rn(__fadd_rn(__fadd_rn(a[g][0], a[g][1]), __fadd_rn(a[g][2], a[g][3])), scale);
            mx[g] = fmaxf(mx[g], s[g]);
        }
        *reinterpret_cast<af4*>(sc + 4 * w) = s;
    }
#pragma unroll
    for (int g = 0; g < kGroup; ++g) {
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) mx[g] = fmaxf(mx[g], __shfl_xor(mx[g], o));
        if (lane == 0) red[wave][g] = mx[g];
    }
    __syncthreads();
    if (tid < kGroup) {
        float m = red[0][tid];
#pragma unroll
        for (int w = 1; w < kAttnThreads / kWave; ++w) m = fmaxf(m, red[w][tid]);
        stat[0][tid] = m;
    }
    __syncthreads();

    // ---- exponentials (elementwise: any thread), then the ordered denominator ----
    for (int i = tid; i < window * kGroup; i += kAttnThreads)
        sc[i] = static_cast<float>(exp(static_cast<double>(__fsub_rn(sc[i], stat[0][i & 3]))));
    __syncthreads();
    if (tid < kGroup) {
        float den = 0.0f;
        int w = 0;
        for (; w + 8 <= window; w += 8) {
            float e[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) e[u] = sc[4 * (w + u) + tid];
#pragma unroll
            for (int u = 0; u < 8; ++u) den = __fadd_rn(den, e[u]);
        }
        for (; w < window; ++w) den = __fadd_rn(den, sc[4 * w + tid]);
        stat[1][tid] = den;
    }
    __syncthreads();
    for (int i = tid; i < window * kGroup; i += kAttnThreads) sc[i] = __fdiv_rn(sc[i], stat[1][i & 3]);
    __syncthreads();

    // ---- values: thread = (dimension d, head pair), keys in order ----
    const int d = tid & (kHeadDim - 1);
    const int g0 = 2 * (tid >> 7);
    const float* vcol = v + static_cast<int64_t>(kh) * kHeadDim + d;
    const int64_t vstride = static_cast<int64_t>(kv_heads) * kHeadDim;
    float o0 = 0.0f, o1 = 0.0f;
    int w = 0;
    for (; w + 8 <= window; w += 8) {
        float vv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) vv[u] = vcol[static_cast<int64_t>(chain[w + u]) * vstride];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            o0 = __fmaf_rn(sc[4 * (w + u) + g0], vv[u], o0);
            o1 = __fmaf_rn(sc[4 * (w + u) + g0 + 1], vv[u], o1);
        }
    }
    for (; w < window; ++w) {
        const float vv = vcol[static_cast<int64_t>(chain[w]) * vstride];
        o0 = __fmaf_rn(sc[4 * w + g0], vv, o0);
        o1 = __fmaf_rn(sc[4 * w + g0 + 1], vv, o1);
    }
    float* orow = out + (row * q_heads + kh * kGroup + g0) * kHeadDim + d;
    orow[0] = o0;
    orow[kHeadDim] = o1;
}

// Packed-sequence attention for head layouts other than GQA-4 (reference
// k_attention, src/tensor.cu:2209-2274, launched by attention_gpu,
// :3316-3340, when q_heads != 4 kv_heads).  One 128-thread workgroup per
// (row, query head); the arithmetic is the reference kernel's:
//   s_w = (fma chain over d ascending of q[d] k_w[d], from +0) * scale
//   m = max_w s_w;  e_w = (float)exp((double)(s_w - m));
//   den = fp32 sum of e_w, w ascending (one lane);  p_w = e_w / den
//   out[d] = fma chain over w ascending of p_w v_w[d]
// The scores and exps of different keys are independent, so threads take
// keys w = tid, tid + 128, ...; only the denominator is a serial sum.  Keys
// are the rows seg_offset[row] + begin .. seg_offset[row] + pos of the row's
// own sequence, begin = max(0, pos + 1 - window).  Dynamic LDS: wmax scores.
constexpr int kAnyThreads = 128;

__global__ void __launch_bounds__(kAnyThreads)
k_attention_any(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
                float* __restrict__ out, const uint32_t* __restrict__ seg_offset, const uint32_t* __restrict__ seg_pos,
                int64_t rows, int q_heads, int kv_heads, int head_dim, int64_t max_seq, int wmax, float scale) {
    extern __shared__ float sc[];
    __shared__ float qs[kAnyThreads];
    __shared__ float red[kAnyThreads / kWave];
    __shared__ float den_s;
    const int tid = threadIdx.x;
    const int64_t task = blockIdx.x;
    const int64_t row = task / q_heads;
    const int qh = static_cast<int>(task % q_heads);
    const int kh = qh / (q_heads / kv_heads);
    // positions and segment starts clamped for memory safety only (the C++
    // layer builds them from the sequence lengths)
    int64_t pos = seg_pos[row];
    pos = pos < max_seq ? pos : max_seq - 1;
    const int64_t begin = pos + 1 > wmax ? pos + 1 - wmax : 0;
    const int window = static_cast<int>(pos - begin + 1);
    const int64_t first = static_cast<int64_t>(seg_offset[row]) + begin;
    auto key_row = [&](int w) {
        const int64_t r = first + w;
        return r < rows ? r : rows - 1;
    };
    const float* qrow = q + (row * q_heads + qh) * static_cast<int64_t>(head_dim);
    if (tid < head_dim) qs[tid] = qrow[tid];
    __syncthreads();
    float m = -3.402823466e+38F;
    for (int w = tid; w < window; w += kAnyThreads) {
        const float* kr = k + (key_row(w) * kv_heads + kh) * static_cast<int64_t>(head_dim);
        float a = 0.0f;
        for (int d = 0; d < head_dim; ++d) a = __fmaf_rn(qs[d], kr[d], a);
        const float sw = __fmul_rn(a, scale);
        sc[w] = sw;
        m = fmaxf(m, sw);
    }
    // the window's maximum (order-independent)
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) m = fmaxf(m, __shfl_xor(m, d));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(red[0], red[1]);
    for (int w = tid; w < window; w += kAnyThreads)
        sc[w] = static_cast<float>(exp(static_cast<double>(__fsub_rn(sc[w], m))));
    __syncthreads();
    if (tid == 0) {
        float den = 0.0f;
        for (int w = 0; w < window; ++w) den = __fadd_rn(den, sc[w]);
        den_s = den;
    }
    __syncthreads();
    const float den = den_s;
    for (int w = tid; w < window; w += kAnyThreads) sc[w] = __fdiv_rn(sc[w], den);
    __syncthreads();
    if (tid < head_dim) {
        float o = 0.0f;
        for (int w = 0; w < window; ++w)
            o = __fmaf_rn(sc[w], v[(key_row(w) * kv_heads + kh) * static_cast<int64_t>(head_dim) + tid], o);
        out[(row * q_heads + qh) * static_cast<int64_t>(head_dim) + tid] = o;
    }
}

}  // namespace

hipError_t launch_rope_tree(float* x, const uint32_t* row_pos, int64_t rows, int heads, int head_dim,
                            const float* cosv, const float* sinv, int64_t max_seq, hipStream_t s) {
    const int64_t pairs = rows * heads * (head_dim / 2);
    if (pairs <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_rope_tree, dim3(static_cast<unsigned>(ceil_div(pairs, 256))), dim3(256), 0, s, x, row_pos,
                       rows, heads, head_dim / 2, cosv, sinv, max_seq);
    return hipGetLastError();
}

hipError_t launch_attention_tree(const float* q, const float* k, const float* v, float* out, const uint32_t* row_pos,
                                 const uint32_t* anc, int64_t anc_stride, int64_t rows, int q_heads, int kv_heads,
                                 int head_dim, int window_max, bool packed, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (head_dim != kHeadDim || q_heads != kGroup * kv_heads || anc_stride <= 0 || window_max <= 0)
        return hipErrorInvalidValue;
    const int64_t keys = anc_stride < window_max ? anc_stride : window_max;
    if (keys > kAttnMaxWindow) return hipErrorInvalidValue;
    const int wmax = static_cast<int>(keys);
    const size_t lds = static_cast<size_t>(wmax) * (kGroup * sizeof(float) + sizeof(uint32_t));
    // dynamic LDS past 64 KB needs the function's limit raised first
    auto kern = packed ? &k_attention_tree<true> : &k_attention_tree<false>;
    if (lds > 65536) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (e != hipSuccess) return e;
    }
    // 1 / sqrtf(head_dim), both correctly rounded, as the reference kernel computes it
    const float root = sqrtf(static_cast<float>(head_dim));
    const float scale = 1.0f / root;
    // path groups on the matrix cores when their scores fit in LDS (16
    // queries x the group's key range) and q, k, v are 16-byte aligned; the
    // rest per row
    const int64_t span = ceil_div(keys + kGroupRows - 1, kKeyTile) * kKeyTile;
    const int sw = static_cast<int>(span) | 1;   // odd row stride: 16 queries, 16 bank groups
    const size_t glds = static_cast<size_t>(kGroupQueries + 1) * sw * sizeof(float);
    const bool group = glds <= 150 * 1024 && rows * kv_heads * kHeadDim * static_cast<int64_t>(sizeof(float)) <= 0xFFFFFFFFll &&
                       ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                         reinterpret_cast<uintptr_t>(v)) & 15u) == 0;
    if (group) {
        // three workgroups per CU (registers trimmed to 168) when three key
        // ranges fit the LDS, else two.  (Splitting one launch into a long-
        // and a short-range launch lost more to the first one's tail than
        // the short ranges gained.)
        const bool three = 3 * (glds + 384) <= 160 * 1024;
        auto gk = three ? (packed ? &k_attention_group<true, 3> : &k_attention_group<false, 3>)
                        : (packed ? &k_attention_group<true, 2> : &k_attention_group<false, 2>);
        if (glds > 65536) {
            const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(gk),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(glds));
            if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL(gk, dim3(static_cast<unsigned>(ceil_div(rows, kGroupRows) * kv_heads)), dim3(256), glds, s,
                           q, k, v, out, row_pos, anc, anc_stride, rows, q_heads, kv_heads, wmax, scale, sw);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(rows * kv_heads)), dim3(kAttnThreads), lds, s, q, k, v, out,
                       row_pos, anc, anc_stride, rows, q_heads, kv_heads, wmax, scale,
                       group ? static_cast<int>(span) : 0);
    return hipGetLastError();
}

hipError_t launch_attention_any(const float* q, const float* k, const float* v, float* out, const uint32_t* seg_offset,
                                const uint32_t* seg_pos, int64_t max_seq, int64_t rows, int q_heads, int kv_heads,
                                int head_dim, int window_max, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (kv_heads <= 0 || q_heads <= 0 || q_heads % kv_heads != 0 || head_dim <= 0 || head_dim > kAnyThreads ||
        max_seq <= 0 || window_max <= 0 || rows * q_heads > 0x7FFFFFFFll)
        return hipErrorInvalidValue;
    const int64_t keys = max_seq < window_max ? max_seq : window_max;
    if (keys > kAttnMaxWindow) return hipErrorInvalidValue;
    const int wmax = static_cast<int>(keys);
    const size_t lds = static_cast<size_t>(wmax) * sizeof(float);
    if (lds > 65536) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_attention_any),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (e != hipSuccess) return e;
    }
    const float root = sqrtf(static_cast<float>(head_dim));
    const float scale = 1.0f / root;
    hipLaunchKernelGGL(k_attention_any, dim3(static_cast<unsigned>(rows * q_heads)), dim3(kAnyThreads), lds, s, q, k,
                       v, out, seg_offset, seg_pos, rows, q_heads, kv_heads, head_dim, max_seq, wmax, scale);
    return hipGetLastError();
}

}  // namespace aps
