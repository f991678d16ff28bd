/* Checks the fp8 row quantiser's division shortcut (aps2026_amd/csrc/quant.hip,
 * quotient()): for a row scale sc = RN(amax / 448) and its reciprocal
 * r = RN(1 / sc), the quotient
 *     q0 = RN(v * r);  q = RN(q0 + RN(v - q0 * sc) * r)   (both fused),
 * given the sign of v (so that -0 stays -0), must give the same e4m3 code as
 * the IEEE quotient RN(v / sc) for every bf16 amax and every bf16 v,
 * |v| <= amax, when sc >= 2^-89 (smaller scales take the IEEE division: then
 * tiny values can have quotients above 2^-10, where an error in the last
 * place of a subnormal residual would show)
 * (a row's values never exceed its amax).  The e4m3 encoder below is the
 * library's (round to nearest even, saturating at 448, subnormal grid 2^-9).
 *
 * usage: quotient_check [stride]   -- v runs over every stride-th bf16 pattern
 *        (stride 1 = exhaustive, 1.07e9 pairs, 90 s); prints the counts and
 *        exits 1 on any mismatch.  The plain product RN(v * r) is counted too,
 *        to show that the correction step is needed. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float f32(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static uint32_t bits(float x) { uint32_t v; memcpy(&v, &x, 4); return v; }

static uint32_t e4m3(float v) {
    const uint32_t sign = (bits(v) >> 24) & 0x80u;
    const float a = fminf(fabsf(v), 448.0f);
    uint32_t code;
    if (a < 0.015625f) {
        code = (uint32_t)nearbyintf(a * 512.0f);
    } else {
        const uint32_t x = bits(a);
        const uint32_t r = x + 0x7FFFFu + ((x >> 20) & 1u);
        code = (((r >> 23) - 127u + 7u) << 3) | ((r >> 20) & 7u);
    }
    return sign | code;
}

int main(int argc, char** argv) {
    const uint32_t stride = argc > 1 ? (uint32_t)atoi(argv[1]) : 1u;
    unsigned long long total = 0, bad = 0, bad_plain = 0;
    for (uint32_t ab = 0; ab < 0x8000u; ++ab) {          /* every non-negative bf16 amax */
        volatile float amax = f32(ab << 16);
        if (isinf(amax) || isnan(amax)) continue;
        float sc = amax / 448.0f;
        if (!(sc > 0.0f)) sc = 1.0f;                     /* an all-zero row */
        volatile float vsc = sc;
        const float r = 1.0f / vsc;
        /* the first pattern of each stride-th block, offset by amax so that
         * every v residue class is visited across amax values */
        for (uint32_t b = ab % stride; b < 0x10000u; b += stride) {
            const float v = f32(b << 16);
            if (isnan(v) || isinf(v) || fabsf(v) > amax) continue;
            volatile float vv = v;
            const uint32_t want = e4m3(vv / vsc);
            float q;
            if (sc < 0x1p-89f) {
                q = vv / vsc;                 /* rows with amax < 2^-80: IEEE division */
            } else {
                const float q0 = v * r;
                q = copysignf(fmaf(fmaf(-q0, sc, v), r, q0), v);
                if (e4m3(q0) != want) ++bad_plain;
            }
            ++total;
            if (e4m3(q) != want) {
                if (bad < 5) printf("mismatch: amax %a v %a\n", (double)amax, (double)v);
                ++bad;
            }
        }
    }
    printf("pairs %llu mismatches %llu plain-product mismatches %llu\n", total, bad, bad_plain);
    return bad != 0;
}
