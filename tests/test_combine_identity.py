"""The fp8 path's folded combine computes the reference's combine of a
token's two bf16 expert outputs, (0 + 0.5 a) + 0.5 b with each step rounded
to fp32 (k_moe_combine, src/tensor.cu:1968-1988), as two FMAs:
fma(a, 0.5, fma(b, 0.5, 0)) (aps2026_amd/csrc/ffn_mfma.hip, combine_fma).
This pins the identity on the CPU for bf16 inputs, over every pair of a set
of special values (signed zeros, subnormals, the normal range's ends,
infinities, NaN) and over random and near-tie pairs.

Emulation: the reference form with numpy float32 arithmetic (correctly
rounded); the FMA form as the float64 sum 0.5 a + t rounded once to float32,
which equals the FMA's single rounding for bf16 inputs: 0.5 a and t carry at
most 8 significant bits, so the float64 sum is exact when their exponents
differ by at most 44, and otherwise the smaller term lies far below half a
float32 ulp of the larger, which both roundings return.
"""
import numpy as np

from aps2026_amd import synth


def bf16(bits):
    return synth.bf16_bits_to_f32(np.asarray(bits, dtype=np.uint16))


def reference(a, b):
    with np.errstate(all="ignore"):
        v = np.float32(0.0) + np.float32(0.5) * a
        return v + np.float32(0.5) * b


def fma_form(a, b):
    with np.errstate(all="ignore"):
        t = (np.float32(0.5) * b).astype(np.float64) + 0.0        # fma(b, 0.5, 0): exact, -0 -> +0
        s = (np.float32(0.5) * a).astype(np.float64) + t          # exact (or far-apart terms)
        return s.astype(np.float32)


def same_bits(x, y):
    nan = np.isnan(x) & np.isnan(y)
    return nan | (x.view(np.uint32) == y.view(np.uint32))


SPECIAL = [0x0000, 0x8000, 0x0001, 0x8001, 0x007F, 0x807F, 0x0080, 0x8080, 0x3F80, 0xBF80, 0x3F81,
           0x7F7F, 0xFF7F, 0x7F80, 0xFF80, 0x7FC0, 0x0100, 0x8100, 0x4000, 0xC000]


def test_special_pairs():
    v = bf16(SPECIAL)
    a, b = np.meshgrid(v, v)
    a, b = a.ravel(), b.ravel()
    assert same_bits(reference(a, b), fma_form(a, b)).all()
    # the reference never yields -0; two -0 terms give +0
    r = reference(np.float32(-0.0), np.float32(-0.0))
    assert r.view(np.uint32) == 0


def test_random_and_near_ties():
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 1 << 16, size=(2, 400_000), dtype=np.uint32).astype(np.uint16)
    a, b = bf16(bits[0]), bf16(bits[1])
    assert same_bits(reference(a, b), fma_form(a, b)).all()
    # magnitudes within a few binades (sums that need rounding), either sign
    e = rng.integers(0x3800, 0x4400, size=200_000)
    m = rng.integers(0, 128, size=(2, 200_000))
    s = rng.integers(0, 2, size=(2, 200_000)) << 15
    a = bf16(((e & 0x7F80) | m[0] | s[0]).astype(np.uint16))
    b = bf16((((e + rng.integers(-256, 256, size=200_000)) & 0x7F80) | m[1] | s[1]).astype(np.uint16))
    assert same_bits(reference(a, b), fma_form(a, b)).all()
