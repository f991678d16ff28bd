// LayerNorm of the decoder layer, the producer of the MoE block's input:
// y = (v - mean) * inv * w + b with v = x (+ residual, written back to x).
//
// Reference: k_layer_norm / k_add_layer_norm (src/tensor.cu:2121-2178) with
// ln_moments, ln_serial_sum, ln_serial_var and ln_write (src/tensor.cu:
// 2032-2119).  Both row sums run on ONE thread in ascending j, because the
// router downstream quantises its logits at 1e-3 with a 2e-2 tie margin and a
// last-ulp change of a LayerNorm output can flip an expert.  The arithmetic,
// operation for operation (nvcc contracts `var += t * t` and `... * w + b`):
//   sum  = fp32 adds of v[j], j ascending       mean = sum / h
//   var  = fma(t, t, var), t = v[j] - mean      inv  = 1 / sqrt(var / h + eps)
//   y[j] = fma((v[j] - mean) * inv, w[j], b[j])
// (this library is built with -ffp-contract=off and IEEE division / square
// root, so every other operation is rounded on its own).
//
// gfx950 mapping.  The sums are dependent chains of h additions: their length,
// not bandwidth, sets the time, and only one lane can own a row.  A wave owns
// 4 rows (lanes 0..3 run their chains), so T = 4096 rows make 1024 one-wave
// workgroups, one per SIMD.  The whole wave stages the rows through LDS in
// chunks of 256 columns: per row one coalesced 1 KB load (64 lanes x 16 B) of
// x (and of the residual, added here and stored back to x), then one 16-byte
// LDS write per lane; the chain lanes read their row four values at a time
// (rows padded by 16 bytes: distinct bank groups).  Loads run kLnDepth chunks
// ahead in a register ring (a chunk's chain, ~0.6 us, is shorter than a load's
// latency), always to a valid address (the last chunk is re-read past the
// end) so that the compiler can count the loads in flight.
//   pass 1: stage x (+ residual), mean chain;
//   pass 2: stage v again (now in x), variance chain;
//   pass 3: y for the 4 rows, coalesced (w and b loaded with each chunk).
#include "common.hpp"

namespace aps {
namespace {

constexpr int kLnRows = 4;      // rows per wave (chain lanes)
constexpr int kLnChunk = 256;   // columns per staged chunk: 1 KB of fp32 per row
constexpr int kLnPitch = kLnChunk + 4;  // staged row pitch in floats (16-byte pad)
constexpr int kLnMaxDepth = 4;  // chunks of loads in flight (NC % depth == 0)

typedef float lf4 __attribute__((ext_vector_type(4)));

template <bool ADD, int kLnDepth>
__global__ void __launch_bounds__(64)
k_layer_norm(float* __restrict__ x, const float* __restrict__ residual, const float* __restrict__ w,
             const float* __restrict__ b, float* __restrict__ y, int64_t rows, int h, float eps) {
    __shared__ __align__(16) float stage[2][kLnRows][kLnPitch];
    __shared__ float s_mean[kLnRows], s_inv[kLnRows];
    const int lane = threadIdx.x;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kLnRows;
    const int nr = rows - r0 < kLnRows ? static_cast<int>(rows - r0) : kLnRows;  // wave-uniform
    const int NC = h / kLnChunk;
    const bool chain = lane < nr;
    // lane's 16-byte piece of row rr, chunk c.  Rows past the end map to the
    // last row (its loads and stores repeat that row's, with equal data), and
    // chunks past the end to the last chunk (loaded ahead, never used), so
    // every load and store is unconditional and the compiler counts them.
    auto piece = [&](const float* base, int rr, int c) -> const lf4* {
        const int64_t row = r0 + (rr < nr ? rr : nr - 1);
        const int cc = c < NC ? c : NC - 1;
        return reinterpret_cast<const lf4*>(base + row * static_cast<int64_t>(h) + cc * kLnChunk) + lane;
    };

    lf4 xs[kLnDepth][kLnRows], rs[kLnDepth][kLnRows];
    auto load = [&](int slot_dummy, lf4 (&xd)[kLnRows], lf4 (&rd)[kLnRows], int c, bool with_residual) {
        (void)slot_dummy;
#pragma unroll
        for (int rr = 0; rr < kLnRows; ++rr) {
            xd[rr] = *piece(x, rr, c);
            if (ADD && with_residual) rd[rr] = *piece(residual, rr, c);
        }
    };
    // v = x (+ residual) into LDS buffer c % 2; pass 1 also writes v back to x
    auto put = [&](const lf4 (&xd)[kLnRows], const lf4 (&rd)[kLnRows], int c, bool with_residual) {
#pragma unroll
        for (int rr = 0; rr < kLnRows; ++rr) {
            lf4 v = xd[rr];
            if (ADD && with_residual) {
                v = lf4{__fadd_rn(v[0], rd[rr][0]), __fadd_rn(v[1], rd[rr][1]), __fadd_rn(v[2], rd[rr][2]),
                        __fadd_rn(v[3], rd[rr][3])};
                *const_cast<lf4*>(piece(x, rr, c)) = v;
            }
            *reinterpret_cast<lf4*>(&stage[c & 1][rr][4 * lane]) = v;
        }
        // every lane stages its pieces, then the chain lanes read whole
        // rows: the wave barrier keeps the compiler from running the two on
        // divergent paths one after the other (a data race between lanes)
        __builtin_amdgcn_wave_barrier();
    };
    // one staged pass over the rows; step(acc, v) folds four values in order
    auto pass = [&](bool with_residual, auto step) {
        float acc = 0.0f;
#pragma unroll
        for (int d = 0; d < kLnDepth; ++d) {
            load(d, xs[d], rs[d], d, with_residual);
            // keep the chunks' loads in order, so that a chunk's wait leaves
            // every later chunk in flight
            __builtin_amdgcn_sched_barrier(0);
        }
        for (int c0 = 0; c0 < NC; c0 += kLnDepth) {
#pragma unroll
            for (int d = 0; d < kLnDepth; ++d) {
                const int c = c0 + d;
                put(xs[d], rs[d], c, with_residual);
                load(d, xs[d], rs[d], c + kLnDepth, with_residual);
                __builtin_amdgcn_sched_barrier(0);
                if (chain) {
                    const float* row = &stage[c & 1][lane][0];
#pragma unroll 8
                    for (int j = 0; j < kLnChunk; j += 4) acc = step(acc, *reinterpret_cast<const lf4*>(row + j));
                }
            }
        }
        return acc;
    };

    // pass 1: the mean (ascending adds)
    const float sum = pass(ADD, [](float a, lf4 v) {
        a = __fadd_rn(a, v[0]);
        a = __fadd_rn(a, v[1]);
        a = __fadd_rn(a, v[2]);
        return __fadd_rn(a, v[3]);
    });
    const float mean = __fdiv_rn(sum, static_cast<float>(h));
    // pass 2: the variance (fused chain of squared deviations); v is in x now,
    // once this wave's stores of pass 1 have completed
    if (ADD) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    const float var = pass(false, [mean](float a, lf4 v) {
        float t = __fsub_rn(v[0], mean);
        a = __fmaf_rn(t, t, a);
        t = __fsub_rn(v[1], mean);
        a = __fmaf_rn(t, t, a);
        t = __fsub_rn(v[2], mean);
        a = __fmaf_rn(t, t, a);
        t = __fsub_rn(v[3], mean);
        return __fmaf_rn(t, t, a);
    });
    if (chain) {
        s_mean[lane] = mean;
        // sqrtf, not __fsqrt_rn: under -fhip-fp32-correctly-rounded-divide-sqrt
        // sqrtf is correctly rounded (v_sqrt_f32 plus a neighbour check),
        // while __fsqrt_rn lowers to the bare v_sqrt_f32, off by an ulp at
        // times (rows of a GPU test disagreed with the oracle by one ulp)
        s_inv[lane] = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(var, static_cast<float>(h)), eps)));
    }
    __syncthreads();
    float m[kLnRows], iv[kLnRows];
#pragma unroll
    for (int rr = 0; rr < kLnRows; ++rr) {
        m[rr] = s_mean[rr];
        iv[rr] = s_inv[rr];
    }

    // pass 3: y, coalesced, loads kLnDepth chunks ahead
    lf4 wv[kLnDepth], bv[kLnDepth];
    auto load_wb = [&](int d, int c) {
        const int cc = c < NC ? c : NC - 1;
        wv[d] = reinterpret_cast<const lf4*>(w + cc * kLnChunk)[lane];
        bv[d] = reinterpret_cast<const lf4*>(b + cc * kLnChunk)[lane];
    };
#pragma unroll
    for (int d = 0; d < kLnDepth; ++d) {
        load(d, xs[d], rs[d], d, false);
        load_wb(d, d);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int c0 = 0; c0 < NC; c0 += kLnDepth) {
#pragma unroll
        for (int d = 0; d < kLnDepth; ++d) {
            const int c = c0 + d;
            lf4 o[kLnRows];
#pragma unroll
            for (int rr = 0; rr < kLnRows; ++rr)
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    o[rr][k] = __fmaf_rn(__fmul_rn(__fsub_rn(xs[d][rr][k], m[rr]), iv[rr]), wv[d][k], bv[d][k]);
            load(d, xs[d], rs[d], c + kLnDepth, false);
            load_wb(d, c + kLnDepth);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int rr = 0; rr < kLnRows; ++rr) {
                const int64_t row = r0 + (rr < nr ? rr : nr - 1);
                *reinterpret_cast<lf4*>(y + row * static_cast<int64_t>(h) + c * kLnChunk + 4 * lane) = o[rr < nr ? rr : nr - 1];
            }
        }
    }
}

}  // namespace

hipError_t launch_layer_norm(float* x, const float* residual, const float* weight, const float* bias, float* y,
                             int64_t rows, int hidden, float eps, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hidden <= 0 || hidden % kLnChunk != 0) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(ceil_div(rows, kLnRows)));
    const int nc = hidden / kLnChunk;
    const int depth = nc % kLnMaxDepth == 0 ? kLnMaxDepth : nc % 2 == 0 ? 2 : 1;
#define APS_LN_LAUNCH(ADD, D)                                                                          \
    hipLaunchKernelGGL((k_layer_norm<ADD, D>), grid, dim3(64), 0, s, x, residual, weight, bias, y, rows, \
                       hidden, eps)
    if (residual) {
        if (depth == 4) APS_LN_LAUNCH(true, 4);
        else if (depth == 2) APS_LN_LAUNCH(true, 2);
        else APS_LN_LAUNCH(true, 1);
    } else {
        if (depth == 4) APS_LN_LAUNCH(false, 4);
        else if (depth == 2) APS_LN_LAUNCH(false, 2);
        else APS_LN_LAUNCH(false, 1);
    }
#undef APS_LN_LAUNCH
    return hipGetLastError();
}

}  // namespace aps
