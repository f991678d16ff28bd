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
// gfx950 mapping: one 256-thread workgroup per (row, KV head) serves the
// four query heads of the group, as in the reference.  Scores: a thread owns
// a key and reads its 128-float row as 16-byte vectors, one element per
// partial sum a_0..a_3 (the four partials are exactly the four lanes of a
// float4), against the four query rows broadcast from LDS.  The
// order-critical denominator runs on four lanes (one per head) of one wave.
// Values: a thread owns one dimension d of two heads and walks the keys in
// order, V rows read coalesced (128 threads = one 512-byte row).
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
                 int64_t anc_stride, int64_t rows, int q_heads, int kv_heads, int wmax, float scale) {
    extern __shared__ __align__(16) float dyn[];
    float* sc = dyn;                                                  // [w][g]
    uint32_t* chain = reinterpret_cast<uint32_t*>(dyn + static_cast<int64_t>(wmax) * kGroup);
    __shared__ __align__(16) float qs[kHeadDim][kGroup];              // [d][g]
    __shared__ float red[kAttnThreads / kWave][kGroup];
    __shared__ float stat[2][kGroup];                                 // max, denominator
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t row = blockIdx.x / kv_heads;
    const int kh = static_cast<int>(blockIdx.x % kv_heads);
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
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(rows * kv_heads)), dim3(kAttnThreads), lds, s, q, k, v, out,
                       row_pos, anc, anc_stride, rows, q_heads, kv_heads, wmax, scale);
    return hipGetLastError();
}

}  // namespace aps
