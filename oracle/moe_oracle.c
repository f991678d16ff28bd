/*
 * CPU oracle for the MoE feed-forward path of ezzy0654/aps2026.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker that the HIP product is
 * compared against, and the CPU baseline timed beside it. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product library (aps2026_amd/) never links, loads or calls anything here.
 *
 * Arithmetic: IEEE-754 binary32, round-to-nearest-even, no flush-to-zero.
 * Built with -ffp-contract=off so that the only fused multiply-adds are the
 * explicit fmaf() calls, which restate the FMA chains the reference's CUDA
 * kernels produce (nvcc contracts `acc += a * b` into one FMA by default).
 *
 * Reference behaviour restated (file:line under the reference tree):
 *   router logits      src/tensor.cu:2957-2998 (k_matmul_transposed_narrow:
 *                      one fp32 accumulator per output, k ascending, +0 init)
 *                      and src/tensor.cu:288-300 (CPU matmul_transposed)
 *   quantise + top-2   src/layer.cu:69-92 (PhiMoE::route),
 *                      src/tensor.cu:1293-1331 (k_moe_top2), constants
 *                      include/config.h:22-23
 *   counts / offsets   src/tensor.cu:1329-1330, 1343-1355
 *   stable permutation src/tensor.cu:1376-1418 (k_moe_fill_stable),
 *                      src/layer.cu:129-134 (assignments[e] in token order)
 *   expert FFN         src/tensor.cu:1925-1965 (gate/up chains + SiLU),
 *                      src/tensor.cu:1799-1835 (w2 chain), src/layer.cu:56-64,
 *                      SiLU src/tensor.cu:284-286, 321-325
 *   combine            src/tensor.cu:1968-1988 (k_moe_combine),
 *                      src/layer.cu:143-146 (zero-initialised y += 0.5 * out)
 *   CPU path order     src/layer.cu:113-148 (PhiMoE::forward, use_gpu=false)
 *
 * How each function is pinned is listed in tests/test_oracle.py; every
 * function here has at least one check that does not restate its formula.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

#define ORACLE_API __attribute__((visibility("default")))

/* Reference constants, include/config.h:22-23. */
#define ORACLE_QUANTUM 1.0e-3f
#define ORACLE_TIE_EPS 2.0e-2f

ORACLE_API int oracle_num_threads(void) { return omp_get_max_threads(); }
ORACLE_API void oracle_set_num_threads(int n) { if (n > 0) omp_set_num_threads(n); }

/* ------------------------------------------------------------------------ */
/* 1. Router logits: logits[t][e] = fma-chain over k ascending of
 *    x[t][k] * gate[e][k], starting from +0.0f.  src/tensor.cu:2957-2998.
 *    The 16 chains of one token run side by side (independent accumulators,
 *    each walked strictly in k order), which lets the compiler vectorise over
 *    e without reordering any chain. */
ORACLE_API int oracle_router_logits(const float* x, const float* gate,
                                    int64_t T, int32_t H, int32_t E,
                                    float* logits) {
    if (T < 0 || H <= 0 || E <= 0 || E > 64) return -1;
    float* gt = (float*)malloc((size_t)H * (size_t)E * sizeof(float));
    if (!gt) return -2;
    for (int32_t e = 0; e < E; ++e)
        for (int32_t k = 0; k < H; ++k) gt[(size_t)k * E + e] = gate[(size_t)e * H + k];
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
        float acc[64];
        for (int32_t e = 0; e < E; ++e) acc[e] = 0.0f;
        const float* xr = x + (size_t)t * H;
        for (int32_t k = 0; k < H; ++k) {
            const float xv = xr[k];
            const float* g = gt + (size_t)k * E;
            for (int32_t e = 0; e < E; ++e) acc[e] = fmaf(xv, g[e], acc[e]);
        }
        for (int32_t e = 0; e < E; ++e) logits[(size_t)t * E + e] = acc[e];
    }
    free(gt);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* 2. Quantise + greedy tie-eps top-2.  src/layer.cu:69-92.
 *    q = sign(l) * floorf(|l| / Q + 0.5f) * Q; a later expert replaces the
 *    incumbent only when q[e] > q[best] + TIE (strictly), so lower indices
 *    win near-ties.  Both picks carry weight 0.5f. */
static int greedy_select(const float* q, int32_t E, int32_t excluded, float tie) {
    int32_t best = -1;
    float best_value = -INFINITY;
    for (int32_t e = 0; e < E; ++e) {
        if (e == excluded) continue;
        if (best < 0 || q[e] > best_value + tie) {
            best = e;
            best_value = q[e];
        }
    }
    return best;
}

ORACLE_API float oracle_quantise(float l, float quantum) {
    const float r = floorf(fabsf(l) / quantum + 0.5f) * quantum;
    return l < 0.0f ? -r : r;
}

ORACLE_API int oracle_route_top2(const float* logits, int64_t T, int32_t E,
                                 float quantum, float tie_eps,
                                 int32_t* routes /* [T][2] */,
                                 float* weights /* [T][2] or NULL */) {
    if (T < 0 || E < 2 || E > 64) return -1;
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
        float q[64];
        for (int32_t e = 0; e < E; ++e) q[e] = oracle_quantise(logits[(size_t)t * E + e], quantum);
        const int32_t first = greedy_select(q, E, -1, tie_eps);
        const int32_t second = greedy_select(q, E, first, tie_eps);
        routes[2 * t] = first;
        routes[2 * t + 1] = second;
        if (weights) {
            weights[2 * t] = 0.5f;
            weights[2 * t + 1] = 0.5f;
        }
    }
    return 0;
}

ORACLE_API float oracle_default_quantum(void) { return ORACLE_QUANTUM; }
ORACLE_API float oracle_default_tie_eps(void) { return ORACLE_TIE_EPS; }

/* ------------------------------------------------------------------------ */
/* 3. Counts, offsets and the stable permutation.
 *    counts[e]  = number of (token, slot) pairs routed to e
 *    offsets    = exclusive scan of counts, offsets[E] = 2T
 *    Expert e's list is its tokens in ascending token order (the CPU path
 *    appends in token order, src/layer.cu:129-134; the GPU fill is a stable
 *    ballot rank, src/tensor.cu:1376-1418).
 *    assignment_rows[offsets[e] + i] = i-th token of e
 *    route_positions[2t + s]         = position of (t, slot s)          */
ORACLE_API int oracle_dispatch(const int32_t* routes, int64_t T, int32_t E,
                               uint32_t* counts, uint32_t* offsets,
                               uint32_t* assignment_rows,
                               uint32_t* route_positions) {
    if (T < 0 || E <= 0) return -1;
    for (int32_t e = 0; e < E; ++e) counts[e] = 0;
    for (int64_t i = 0; i < 2 * T; ++i) {
        const int32_t e = routes[i];
        if (e < 0 || e >= E) return -3;
        counts[e]++;
    }
    offsets[0] = 0;
    for (int32_t e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    uint32_t* cursor = (uint32_t*)malloc((size_t)E * sizeof(uint32_t));
    if (!cursor) return -2;
    for (int32_t e = 0; e < E; ++e) cursor[e] = offsets[e];
    for (int64_t t = 0; t < T; ++t) {
        for (int s = 0; s < 2; ++s) {
            const int32_t e = routes[2 * t + s];
            const uint32_t pos = cursor[e]++;
            assignment_rows[pos] = (uint32_t)t;
            route_positions[2 * t + s] = pos;
        }
    }
    free(cursor);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* 4. Expert FFN for a list of (row, expert) pairs.
 *      g_j = fma-chain_k x[k] * w1[e][j][k]      (k ascending, +0 init)
 *      u_j = fma-chain_k x[k] * w3[e][j][k]
 *      a_j = (g_j / (1 + (float)exp((double)-g_j))) * u_j
 *      y_i = fma-chain_j a_j * w2[e][i][j]       (j ascending, +0 init)
 *    src/tensor.cu:1925-1965 and 1799-1835; SiLU src/tensor.cu:284-286.
 *    Weights are transposed once per call so that the inner loop runs over
 *    independent output chains; no chain is reordered. */
static inline float silu_mul(float g, float u) {
    const float ex = (float)exp((double)(-g));
    const float s = g / (1.0f + ex);
    return s * u;
}

ORACLE_API int oracle_ffn_rows(const float* xrows /* [n][H] */,
                               const int32_t* experts /* [n] */, int64_t n,
                               int32_t H, int32_t F, int32_t E,
                               const float* w1 /* [E][F][H] */,
                               const float* w3 /* [E][F][H] */,
                               const float* w2 /* [E][H][F] */,
                               float* act /* [n][F] or NULL */,
                               float* y /* [n][H] */) {
    if (n < 0 || H <= 0 || F <= 0 || E <= 0) return -1;
    for (int64_t r = 0; r < n; ++r)
        if (experts[r] < 0 || experts[r] >= E) return -3;
    /* Which experts are used, so only those are transposed. */
    char* used = (char*)calloc((size_t)E, 1);
    if (!used) return -2;
    for (int64_t r = 0; r < n; ++r) used[experts[r]] = 1;
    const size_t fh = (size_t)F * (size_t)H;
    float* w1t = (float*)malloc(fh * (size_t)E * sizeof(float)); /* [E][H][F] */
    float* w3t = (float*)malloc(fh * (size_t)E * sizeof(float)); /* [E][H][F] */
    float* w2t = (float*)malloc(fh * (size_t)E * sizeof(float)); /* [E][F][H] */
    float* abuf = act ? NULL : (float*)malloc((size_t)(n > 0 ? n : 1) * (size_t)F * sizeof(float));
    if (!w1t || !w3t || !w2t || (!act && !abuf)) {
        free(used); free(w1t); free(w3t); free(w2t); free(abuf);
        return -2;
    }
    float* a_out = act ? act : abuf;
#pragma omp parallel for collapse(2) schedule(static)
    for (int32_t e = 0; e < E; ++e) {
        for (int32_t j = 0; j < F; ++j) {
            if (!used[e]) continue;
            const float* s1 = w1 + (size_t)e * fh + (size_t)j * H;
            const float* s3 = w3 + (size_t)e * fh + (size_t)j * H;
            float* d1 = w1t + (size_t)e * fh;
            float* d3 = w3t + (size_t)e * fh;
            for (int32_t k = 0; k < H; ++k) {
                d1[(size_t)k * F + j] = s1[k];
                d3[(size_t)k * F + j] = s3[k];
            }
            for (int32_t i = 0; i < H; ++i)
                w2t[(size_t)e * fh + (size_t)j * H + i] = w2[(size_t)e * fh + (size_t)i * F + j];
        }
    }
    /* Rows are processed in blocks of up to RB consecutive rows that share an
     * expert, so each weight column is swept once per block; every output
     * still has its own accumulator walked in ascending k (or j). */
    enum { RB = 8 };
    int64_t nblocks = 0;
    int64_t* bstart = (int64_t*)malloc((size_t)(n > 0 ? n : 1) * sizeof(int64_t));
    if (!bstart) { free(used); free(w1t); free(w3t); free(w2t); free(abuf); return -2; }
    for (int64_t r = 0; r < n;) {
        int64_t len = 1;
        while (r + len < n && len < RB && experts[r + len] == experts[r]) ++len;
        bstart[nblocks++] = r;
        r += len;
    }
#pragma omp parallel
    {
        float* g = (float*)malloc((size_t)RB * F * sizeof(float));
        float* u = (float*)malloc((size_t)RB * F * sizeof(float));
        float* acc = (float*)malloc((size_t)RB * H * sizeof(float));
#pragma omp for schedule(dynamic, 1)
        for (int64_t b = 0; b < nblocks; ++b) {
            const int64_t r0 = bstart[b];
            const int32_t e = experts[r0];
            int64_t nr = 1;
            while (r0 + nr < n && nr < RB && experts[r0 + nr] == e) ++nr;
            const float* a1 = w1t + (size_t)e * fh;
            const float* a3 = w3t + (size_t)e * fh;
            for (int64_t i = 0; i < nr * F; ++i) { g[i] = 0.0f; u[i] = 0.0f; }
            for (int32_t k = 0; k < H; ++k) {
                const float* c1 = a1 + (size_t)k * F;
                const float* c3 = a3 + (size_t)k * F;
                for (int64_t r = 0; r < nr; ++r) {
                    const float xv = xrows[(size_t)(r0 + r) * H + k];
                    float* gr = g + (size_t)r * F;
                    float* ur = u + (size_t)r * F;
                    for (int32_t j = 0; j < F; ++j) {
                        gr[j] = fmaf(xv, c1[j], gr[j]);
                        ur[j] = fmaf(xv, c3[j], ur[j]);
                    }
                }
            }
            for (int64_t r = 0; r < nr; ++r) {
                float* ar = a_out + (size_t)(r0 + r) * F;
                for (int32_t j = 0; j < F; ++j) ar[j] = silu_mul(g[(size_t)r * F + j], u[(size_t)r * F + j]);
            }
            const float* b2 = w2t + (size_t)e * fh;
            for (int64_t i = 0; i < nr * H; ++i) acc[i] = 0.0f;
            for (int32_t j = 0; j < F; ++j) {
                const float* c2 = b2 + (size_t)j * H;
                for (int64_t r = 0; r < nr; ++r) {
                    const float av = a_out[(size_t)(r0 + r) * F + j];
                    float* accr = acc + (size_t)r * H;
                    for (int32_t i = 0; i < H; ++i) accr[i] = fmaf(av, c2[i], accr[i]);
                }
            }
            memcpy(y + (size_t)r0 * H, acc, (size_t)nr * H * sizeof(float));
        }
        free(g); free(u); free(acc);
    }
    free(bstart);
    free(used); free(w1t); free(w3t); free(w2t); free(abuf);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* 5. Combine: out[t][d] = RN(0.5f * y[p_lo][d] + 0.5f * y[p_hi][d]), lo/hi
 *    ordered by expert id (src/tensor.cu:1968-1988).  0.5f * v is exact, so
 *    the sum rounds once and the order cannot change bits; the expert order
 *    is kept anyway to follow the reference literally. */
ORACLE_API int oracle_combine(const float* y /* [2T][H] */,
                              const int32_t* routes, const uint32_t* route_positions,
                              int64_t T, int32_t H, float* out /* [T][H] */) {
    if (T < 0 || H <= 0) return -1;
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
        const int32_t e0 = routes[2 * t], e1 = routes[2 * t + 1];
        uint32_t p_lo = route_positions[2 * t], p_hi = route_positions[2 * t + 1];
        if (e1 < e0) { const uint32_t tmp = p_lo; p_lo = p_hi; p_hi = tmp; }
        const float* a = y + (size_t)p_lo * H;
        const float* b = y + (size_t)p_hi * H;
        float* o = out + (size_t)t * H;
        for (int32_t d = 0; d < H; ++d) {
            float v = 0.0f;
            v += 0.5f * a[d];
            v += 0.5f * b[d];
            o[d] = v;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* 6. The whole block in the reference CPU path's order
 *    (src/layer.cu:113-148): router GEMM, route every token, then for each
 *    expert in ascending order gather its rows, run the expert MLP and
 *    scatter-add 0.5 * output into a zero-initialised y.  This is the
 *    "reference algorithm's CPU path" that bench.py times as cpu_baseline.
 *    Outputs of the intermediate stages are optional (NULL = not wanted). */
ORACLE_API int oracle_moe_forward(const float* x, const float* gate,
                                  const float* w1, const float* w3, const float* w2,
                                  int64_t T, int32_t H, int32_t F, int32_t E,
                                  float* out /* [T][H] */,
                                  float* logits_out /* [T][E] or NULL */,
                                  int32_t* routes_out /* [T][2] or NULL */) {
    if (T < 0 || H <= 0 || F <= 0 || E < 2 || E > 64) return -1;
    int rc = 0;
    float* logits = (float*)malloc((size_t)(T > 0 ? T : 1) * E * sizeof(float));
    int32_t* routes = (int32_t*)malloc((size_t)(T > 0 ? T : 1) * 2 * sizeof(int32_t));
    int64_t* rows = (int64_t*)malloc((size_t)(T > 0 ? T : 1) * sizeof(int64_t));
    if (!logits || !routes || !rows) { rc = -2; goto done; }
    if ((rc = oracle_router_logits(x, gate, T, H, E, logits))) goto done;
    if ((rc = oracle_route_top2(logits, T, E, ORACLE_QUANTUM, ORACLE_TIE_EPS, routes, NULL))) goto done;
    memset(out, 0, (size_t)T * H * sizeof(float));
    for (int32_t e = 0; e < E; ++e) {
        int64_t count = 0;
        for (int64_t t = 0; t < T; ++t)
            if (routes[2 * t] == e || routes[2 * t + 1] == e) rows[count++] = t;
        if (!count) continue;
        float* xin = (float*)malloc((size_t)count * H * sizeof(float));
        float* yout = (float*)malloc((size_t)count * H * sizeof(float));
        int32_t* ex = (int32_t*)malloc((size_t)count * sizeof(int32_t));
        if (!xin || !yout || !ex) { free(xin); free(yout); free(ex); rc = -2; goto done; }
        for (int64_t i = 0; i < count; ++i) {
            memcpy(xin + (size_t)i * H, x + (size_t)rows[i] * H, (size_t)H * sizeof(float));
            ex[i] = e;
        }
        rc = oracle_ffn_rows(xin, ex, count, H, F, E, w1, w3, w2, NULL, yout);
        if (!rc) {
#pragma omp parallel for schedule(static)
            for (int64_t i = 0; i < count; ++i) {
                float* o = out + (size_t)rows[i] * H;
                const float* v = yout + (size_t)i * H;
                for (int32_t d = 0; d < H; ++d) o[d] += 0.5f * v[d];
            }
        }
        free(xin); free(yout); free(ex);
        if (rc) goto done;
    }
    if (logits_out) memcpy(logits_out, logits, (size_t)T * E * sizeof(float));
    if (routes_out) memcpy(routes_out, routes, (size_t)T * 2 * sizeof(int32_t));
done:
    free(logits); free(routes); free(rows);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* 7. Dtype helpers used to build the exact upcasts the oracle consumes.
 *    bf16 -> fp32 is a 16-bit shift (exact).  fp8 e4m3 (OCP "fn" variant:
 *    bias 7, no infinities, 0x7f/0xff are NaN, max 448) -> fp32 is exact. */
ORACLE_API void oracle_bf16_to_f32(const uint16_t* src, float* dst, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const uint32_t b = (uint32_t)src[i] << 16;
        float f;
        memcpy(&f, &b, 4);
        dst[i] = f;
    }
}

static float e4m3_to_f32(uint8_t v) {
    const int s = v >> 7, e = (v >> 3) & 0xf, m = v & 7;
    float r;
    if (e == 0xf && m == 7) return NAN;
    if (e == 0) r = ldexpf((float)m, -9); /* subnormal: m * 2^-3 * 2^-6 */
    else r = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return s ? -r : r;
}

ORACLE_API void oracle_e4m3_to_f32(const uint8_t* src, float* dst, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) dst[i] = e4m3_to_f32(src[i]);
}

/* e4m3 code of a finite float: the nearest of the 253 finite e4m3 values,
 * ties to the even code (even mantissa), saturating at +-448.  Written from
 * the format definition: between 2^e and 2^(e+1) (e >= -6) the spacing is
 * 2^(e-3); below 2^-6 it is 2^-9. */
static uint8_t f32_to_e4m3(float v) {
    const uint8_t sign = signbit(v) ? 0x80 : 0x00;
    double a = fabs((double)v);
    if (a > 448.0) a = 448.0;
    int e;
    (void)frexp(a, &e);                    /* a = f * 2^e, f in [0.5, 1) */
    int ue = e - 1;                        /* a in [2^ue, 2^(ue+1)) */
    if (ue < -6) ue = -6;
    const double step = ldexp(1.0, ue - 3);
    double q = nearbyint(a / step) * step; /* current rounding mode: to nearest even */
    if (q > 448.0) q = 448.0;
    if (q < ldexp(1.0, -6)) return (uint8_t)(sign | (uint8_t)nearbyint(q / ldexp(1.0, -9)));
    int qe;
    (void)frexp(q, &qe);
    qe -= 1;
    const int mant = (int)nearbyint(q / ldexp(1.0, qe) * 8.0) - 8;
    return (uint8_t)(sign | ((qe + 7) << 3) | mant);
}

/* Per-row e4m3 quantisation of rows x n (the fp8 path's activation format):
 * scale[r] = fp32(amax / 448) (1 if the row is zero), codes = e4m3(fp32(v /
 * scale)), each division rounded to fp32 first. */
ORACLE_API void oracle_quantise_rows_e4m3(const float* src, int64_t rows, int32_t n, uint8_t* codes,
                                          float* scale) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* row = src + r * n;
        float amax = 0.0f;
        for (int32_t k = 0; k < n; ++k) amax = fmaxf(amax, fabsf(row[k]));
        volatile float sc = amax / 448.0f;
        float s = sc > 0.0f ? sc : 1.0f;
        scale[r] = s;
        for (int32_t k = 0; k < n; ++k) {
            volatile float q = row[k] / s;
            codes[r * n + k] = f32_to_e4m3(q);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* LayerNorm of the decoder layer (the MoE block's input), GPU-path semantics:
 * src/tensor.cu:2144-2178 (k_add_layer_norm: v = x + residual, written back
 * to x), src/tensor.cu:2121-2140 (k_layer_norm), with ln_moments / ln_serial_sum
 * / ln_serial_var / ln_write at src/tensor.cu:2056-2119 and 2032-2055:
 *   sum  = fp32 adds of v[j], j ascending, +0 init      mean = sum / h
 *   var  = fma(t, t, var), t = v[j] - mean, j ascending (nvcc contracts
 *          `var += t * t`), +0 init
 *   inv  = 1 / sqrtf(var / h + eps)     (IEEE division and square root)
 *   y[j] = fma((v[j] - mean) * inv, w[j], b[j])   (`... * w + b` contracted)
 * The CPU twin (src/tensor.cu:327-341) sums in the same order.  x_out
 * (optional) receives v; residual may be NULL (plain LayerNorm).  mean_out and
 * inv_out (optional) receive the row statistics. */
ORACLE_API void oracle_layer_norm(const float* x, const float* residual, int64_t rows, int32_t h,
                                  const float* w, const float* b, float eps, float* x_out, float* y,
                                  float* mean_out, float* inv_out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * h;
        const float* rr = residual ? residual + r * h : NULL;
        float* vr = x_out ? x_out + r * h : NULL;
        float sum = 0.0f;
        for (int32_t j = 0; j < h; ++j) {
            const float v = rr ? xr[j] + rr[j] : xr[j];
            if (vr) vr[j] = v;
            sum += v;
        }
        const float mean = sum / (float)h;
        float var = 0.0f;
        for (int32_t j = 0; j < h; ++j) {
            const float v = rr ? xr[j] + rr[j] : xr[j];
            const float t = v - mean;
            var = fmaf(t, t, var);
        }
        const float inv = 1.0f / sqrtf(var / (float)h + eps);
        if (mean_out) mean_out[r] = mean;
        if (inv_out) inv_out[r] = inv;
        for (int32_t j = 0; j < h; ++j) {
            const float v = rr ? xr[j] + rr[j] : xr[j];
            const float a = (v - mean) * inv;
            y[r * h + j] = fmaf(a, w[j], b[j]);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Tree attention of the prefix-deduplicated rows (scope row f4).
 *
 * RoPE table, reference src/tensor.cu:2703-2735 (host code, float
 * arithmetic through std::pow / std::cos / std::sin on floats, i.e. glibc's
 * powf / cosf / sinf):
 *   inv = powf(theta, (-2.0f * j) / head_dim);  cos[p][j] = cosf(p * inv),
 *   sin[p][j] = sinf(p * inv)                  (p * inv rounded to float)
 * RoPE, src/tensor.cu:2180-2197 (k_rope), pair (j, j + half) of each head at
 * the row's position:
 *   x0' = fma(x0, c, -(x1 * s)),  x1' = fma(x1, c, x0 * s)
 * (the reference's `x0 * c - x1 * s` and `x1 * c + x0 * s` as contracted by
 * the LLVM rule that fuses the left product; which product nvcc fuses is not
 * fixed by the source: parity unpinned at that last rounding).
 * Attention, src/tensor.cu:2407-2633 (k_attention_tree_gqa4), per row, KV
 * head kh and query head qh = 4 kh + g:
 *   pos = row_pos[row]; begin = pos + 1 > window_max ? pos + 1 - window_max : 0
 *   key w (0 <= w <= pos - begin) is row anc[row][begin + w]
 *   a_j = fma chain over d = j, j + 4, ... ascending of q[d] * k[d]  (j < 4)
 *   s_w = ((a_0 + a_1) + (a_2 + a_3)) * (1 / sqrtf(head_dim))
 *   m = max_w s_w;  e_w = (float)exp((double)(s_w - m))
 *   den = fp32 sum of e_w, w ascending;  p_w = e_w / den
 *   out[d] = fma chain over w ascending of p_w * v[key w][d]
 * exp is glibc's double exp here and ROCm's in the kernel (the reference:
 * CUDA's): all within an ulp of double, so the float results agree except in
 * the rare case of a double within an ulp of a float rounding boundary. */
ORACLE_API void oracle_rope_table(int64_t max_seq, int32_t head_dim, float theta, float* cosv, float* sinv) {
    const int32_t half = head_dim / 2;
    for (int64_t p = 0; p < max_seq; ++p)
        for (int32_t j = 0; j < half; ++j) {
            volatile float ex = (-2.0f * (float)j) / (float)head_dim;
            const float inv = powf(theta, ex);
            volatile float ang = (float)p * inv;
            cosv[p * half + j] = cosf(ang);
            sinv[p * half + j] = sinf(ang);
        }
}

ORACLE_API void oracle_rope_tree(float* x, const uint32_t* row_pos, int64_t rows, int32_t heads, int32_t head_dim,
                                 const float* cosv, const float* sinv) {
    const int32_t half = head_dim / 2;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r)
        for (int32_t h = 0; h < heads; ++h) {
            float* base = x + (r * heads + h) * (int64_t)head_dim;
            const int64_t t = (int64_t)row_pos[r] * half;
            for (int32_t j = 0; j < half; ++j) {
                const float c = cosv[t + j], s = sinv[t + j];
                const float x0 = base[j], x1 = base[j + half];
                volatile float x1s = x1 * s, x0s = x0 * s;
                base[j] = fmaf(x0, c, -x1s);
                base[j + half] = fmaf(x1, c, x0s);
            }
        }
}

ORACLE_API void oracle_attention_tree(const float* q, const float* k, const float* v, float* out,
                                      const uint32_t* row_pos, const uint32_t* anc, int64_t anc_stride, int64_t rows,
                                      int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t window_max) {
    volatile float root = sqrtf((float)head_dim);
    const float scale = 1.0f / root;
    const int32_t group = q_heads / kv_heads;
#pragma omp parallel
    {
        float* e = (float*)malloc(sizeof(float) * (size_t)(window_max > 0 ? window_max : 1));
#pragma omp for schedule(dynamic, 4)
        for (int64_t row = 0; row < rows; ++row) {
            const int64_t pos = row_pos[row];
            const int64_t begin = pos + 1 > window_max ? pos + 1 - window_max : 0;
            const int64_t window = pos - begin + 1;
            const uint32_t* chain = anc + row * anc_stride + begin;
            for (int32_t qh = 0; qh < q_heads; ++qh) {
                const int32_t kh = qh / group;
                const float* qv = q + (row * q_heads + qh) * (int64_t)head_dim;
                float m = -3.402823466e+38F;
                for (int64_t w = 0; w < window; ++w) {
                    const float* kv = k + ((int64_t)chain[w] * kv_heads + kh) * head_dim;
                    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                    for (int32_t d = 0; d < head_dim; ++d) a[d & 3] = fmaf(qv[d], kv[d], a[d & 3]);
                    volatile float s01 = a[0] + a[1], s23 = a[2] + a[3];
                    volatile float s = s01 + s23;
                    e[w] = s * scale;
                    m = fmaxf(m, e[w]);
                }
                float den = 0.0f;
                for (int64_t w = 0; w < window; ++w) {
                    volatile float t = e[w] - m;
                    e[w] = (float)exp((double)t);
                    den += e[w];
                }
                for (int64_t w = 0; w < window; ++w) e[w] = e[w] / den;
                float* o = out + (row * q_heads + qh) * (int64_t)head_dim;
                for (int32_t d = 0; d < head_dim; ++d) {
                    float val = 0.0f;
                    for (int64_t w = 0; w < window; ++w)
                        val = fmaf(e[w], v[((int64_t)chain[w] * kv_heads + kh) * head_dim + d], val);
                    o[d] = val;
                }
            }
        }
        free(e);
    }
}

/* Packed-sequence attention for head layouts other than GQA-4 (reference
 * k_attention, src/tensor.cu:2209-2274, launched by attention_gpu :3316-3340
 * when q_heads != 4 kv_heads).  Row r sits at position seg_pos[r] of the
 * sequence starting at row seg_offset[r]; its keys are rows seg_offset[r] +
 * begin .. seg_offset[r] + pos, begin = max(0, pos + 1 - window_max).  Per
 * (row, query head qh), kv head kh = qh / (q_heads / kv_heads):
 *   s_w = (fma chain over d ascending of q[d] k_w[d], from +0) * scale,
 *         scale = 1 / sqrtf(head_dim)
 *   m = fmaxf over w from -FLT_MAX;  e_w = (float)exp((double)(s_w - m))
 *   den = fp32 sum of e_w, w ascending;  p_w = e_w / den
 *   out[d] = fma chain over w ascending of p_w v_w[d]
 * (The GQA-4 kernel scores with four partial sums instead, see
 * oracle_attention_tree.) */
ORACLE_API void oracle_attention_generic(const float* q, const float* k, const float* v, float* out,
                                         const uint32_t* seg_offset, const uint32_t* seg_pos, int64_t rows,
                                         int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t window_max) {
    volatile float root = sqrtf((float)head_dim);
    const float scale = 1.0f / root;
    const int32_t group = q_heads / kv_heads;
#pragma omp parallel
    {
        float* e = (float*)malloc(sizeof(float) * (size_t)(window_max > 0 ? window_max : 1));
#pragma omp for schedule(dynamic, 4)
        for (int64_t row = 0; row < rows; ++row) {
            const int64_t pos = seg_pos[row];
            const int64_t begin = pos + 1 > window_max ? pos + 1 - window_max : 0;
            const int64_t window = pos - begin + 1;
            const int64_t first = (int64_t)seg_offset[row] + begin;
            for (int32_t qh = 0; qh < q_heads; ++qh) {
                const int32_t kh = qh / group;
                const float* qv = q + (row * q_heads + qh) * (int64_t)head_dim;
                float m = -3.402823466e+38F;
                for (int64_t w = 0; w < window; ++w) {
                    const float* kv = k + ((first + w) * kv_heads + kh) * (int64_t)head_dim;
                    float a = 0.0f;
                    for (int32_t d = 0; d < head_dim; ++d) a = fmaf(qv[d], kv[d], a);
                    volatile float sw = a * scale;
                    e[w] = sw;
                    m = fmaxf(m, e[w]);
                }
                float den = 0.0f;
                for (int64_t w = 0; w < window; ++w) {
                    volatile float t = e[w] - m;
                    e[w] = (float)exp((double)t);
                    den += e[w];
                }
                for (int64_t w = 0; w < window; ++w) e[w] = e[w] / den;
                float* o = out + (row * q_heads + qh) * (int64_t)head_dim;
                for (int32_t d = 0; d < head_dim; ++d) {
                    float val = 0.0f;
                    for (int64_t w = 0; w < window; ++w)
                        val = fmaf(e[w], v[((first + w) * kv_heads + kh) * (int64_t)head_dim + d], val);
                    o[d] = val;
                }
            }
        }
        free(e);
    }
}

/* Linear layer, GPU-path semantics: src/layer.cu:30-42 (Linear::forward) ->
 * src/tensor.cu:3120-3143 (matmul_transposed_bias_gpu) -> k_matmul_transposed_8x8
 * (src/tensor.cu:715-800): y[t][n] = (fp32 FMA chain over k ascending of
 * x[t][k] * w[n][k], +0 init) + bias[n] (one rounded add; none without a
 * bias).  The same chain as oracle_router_logits for any output count. */
ORACLE_API int oracle_linear(const float* x, const float* w, const float* bias, int64_t T, int32_t K, int32_t N,
                             float* y) {
    if (T < 0 || K <= 0 || N <= 0) return -1;
    float* wt = (float*)malloc((size_t)K * (size_t)N * sizeof(float));
    if (!wt) return -2;
    for (int32_t n = 0; n < N; ++n)
        for (int32_t k = 0; k < K; ++k) wt[(size_t)k * N + n] = w[(size_t)n * K + k];
    int rc = 0;
#pragma omp parallel
    {
        float* acc = (float*)malloc((size_t)N * sizeof(float));
        if (!acc) {
#pragma omp atomic write
            rc = -2;
        } else {
#pragma omp for schedule(static)
            for (int64_t t = 0; t < T; ++t) {
                for (int32_t n = 0; n < N; ++n) acc[n] = 0.0f;
                const float* xr = x + (size_t)t * K;
                for (int32_t k = 0; k < K; ++k) {
                    const float xv = xr[k];
                    const float* g = wt + (size_t)k * N;
                    for (int32_t n = 0; n < N; ++n) acc[n] = fmaf(xv, g[n], acc[n]);
                }
                for (int32_t n = 0; n < N; ++n) y[(size_t)t * N + n] = bias ? acc[n] + bias[n] : acc[n];
            }
            free(acc);
        }
    }
    free(wt);
    return rc;
}
