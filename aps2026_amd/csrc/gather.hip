// Row gather out[i] = x[rows[i]] (fp32 rows of `hidden` values), the
// embedding lookup of the prefix-deduplicated prompt rows and the
// last-token gather before the LM head.
//
// Reference: k_gather_rows (src/tensor.cu:2635-2642) behind
// tensor_ops::gather_rows_gpu (src/tensor.cu:3379-3386 and 3420-3426), one
// thread per element.  Here a 256-thread workgroup copies a 4096-value span
// of one row: each thread issues its four 16-byte loads before any store, so
// a CU with eight workgroups keeps 128 KB of reads in flight, and the kernel runs
// at HBM speed (2 x count x hidden x 4 bytes).  An index past the end of x
// yields a zero row instead of a read out of bounds (the reference does not
// check; the C++ and Python layers reject such indices on the host).
#include "common.hpp"

namespace aps {
namespace {

constexpr int kGatherThreads = 256;
// values of one row per workgroup: four per thread, as 16-byte vectors or
// single floats
template <bool VEC>
constexpr int gather_span() { return kGatherThreads * 4 * (VEC ? 4 : 1); }

typedef float gf4 __attribute__((ext_vector_type(4)));

// VEC: hidden % 4 == 0 and 16-byte aligned arrays (16-byte accesses).
template <bool VEC>
__global__ void __launch_bounds__(kGatherThreads)
k_gather_rows(const float* __restrict__ x, int64_t x_rows, int64_t h, const uint32_t* __restrict__ rows,
              float* __restrict__ out, int64_t spans_per_row) {
    const int64_t b = blockIdx.x;
    const int64_t i = b / spans_per_row;
    const int64_t c0 = (b - i * spans_per_row) * gather_span<VEC>();
    const uint32_t r = rows[i];
    const bool valid = r < static_cast<uint64_t>(x_rows);
    const float* src = x + (valid ? static_cast<int64_t>(r) : 0) * h;
    float* dst = out + i * h;
    const int tid = threadIdx.x;
    if constexpr (VEC) {
        gf4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t c = c0 + 4 * (tid + kGatherThreads * k);
            v[k] = valid && c < h ? *reinterpret_cast<const gf4*>(src + c) : gf4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t c = c0 + 4 * (tid + kGatherThreads * k);
            if (c < h) *reinterpret_cast<gf4*>(dst + c) = v[k];
        }
    } else {
        float v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t c = c0 + tid + kGatherThreads * k;
            v[k] = valid && c < h ? src[c] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t c = c0 + tid + kGatherThreads * k;
            if (c < h) dst[c] = v[k];
        }
    }
}

}  // namespace

hipError_t launch_gather_rows(const float* x, int64_t x_rows, int64_t hidden, const uint32_t* rows, int64_t count,
                              float* out, hipStream_t s) {
    if (count <= 0 || hidden <= 0) return hipSuccess;
    const bool vec = hidden % 4 == 0 &&
                     ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) & 15u) == 0;
    const int64_t spans = ceil_div(hidden, vec ? gather_span<true>() : gather_span<false>());
    const int64_t blocks = count * spans;
    if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
    if (vec)
        hipLaunchKernelGGL(k_gather_rows<true>, dim3(static_cast<unsigned>(blocks)), dim3(kGatherThreads), 0, s, x,
                           x_rows, hidden, rows, out, spans);
    else
        hipLaunchKernelGGL(k_gather_rows<false>, dim3(static_cast<unsigned>(blocks)), dim3(kGatherThreads), 0, s, x,
                           x_rows, hidden, rows, out, spans);
    return hipGetLastError();
}

}  // namespace aps
