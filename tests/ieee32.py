"""Exact IEEE-754 binary32 arithmetic on Python Fractions (round to nearest,
ties to even, no flush).  An arithmetic engine independent of the C compiler
and of numpy, used to check the oracle's router rule on random inputs."""
from fractions import Fraction as Fr
import math
import struct


def f32(x) -> Fr:
    """Round an exact rational to the nearest binary32 value (normals and
    subnormals; |x| below 2^-126 uses the subnormal spacing 2^-149)."""
    x = Fr(x)
    if x == 0:
        return Fr(0)
    s = -1 if x < 0 else 1
    a = abs(x)
    e = math.floor(math.log2(a))
    while Fr(2) ** e > a:
        e -= 1
    while Fr(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)
    ulp = Fr(2) ** (e - 23)
    q, r = divmod(a, ulp)
    if r * 2 > ulp or (r * 2 == ulp and q % 2 == 1):
        q += 1
    return s * q * ulp


def from_float(v: float) -> Fr:
    """Exact value of a Python float already representable in binary32."""
    return Fr(struct.unpack("f", struct.pack("f", v))[0])


def to_float(v: Fr) -> float:
    return float(v)
