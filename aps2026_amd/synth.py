"""Deterministic synthetic inputs for the MoE feed-forward block.

Shapes follow the reference model (include/config.h:8,13-15 of the reference:
hidden 4096, 16 experts, top-2, expert FFN 448) and its weight storage, which
is nn.Linear's ``[out, in]``: ``gate [E, H]``, ``w1, w3 [E, F, H]``,
``w2 [E, H, F]`` (reference src/layer.cu:44-47, 94-99).

Every array comes from one ``numpy.random.default_rng(seed)`` (PCG64) stream
drawn in a fixed order, so the same seed gives the same bits on any x86 host
with this numpy.  Values are always returned as float32 arrays holding the
*exact* values the device computes with (bf16 / fp8 inputs are stored as
their exact fp32 upcasts), plus the packed device encodings.

Skewed expert loads (configs C2 and C5) are produced without changing the
reference's bias-free router (src/layer.cu:96,116): column H-1 of x is set to
1.0 and column H-1 of the gate to a per-expert bias b_e.  The router's FMA
chain then adds b_e exactly in its last step.  The b_e table below was
calibrated once, offline (tests/golden/calibrate_zipf.py), so that the
assignment shares follow Zipf(s=1.1) under the reference routing rule.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Optional

import numpy as np

HIDDEN = 4096
NUM_EXPERTS = 16
FFN = 448
TOP_K = 2
WEIGHT_STD = 0.02
FP8_E4M3_MAX = 448.0

# Per-expert router bias for Zipf(1.1) assignment shares with 16 experts,
# H = 4096, gate ~ N(0, 0.02), x ~ N(0, 1).  Written by
# tests/golden/calibrate_zipf.py; exact float32 values.
ZIPF_1_1_BIAS = np.array([
    2.129412889480591, 1.0321242809295654, 0.6186558604240417, 0.3333785831928253,
    0.1317485272884369, 0.011133951134979725, -0.1081472709774971, -0.2324112206697464,
    -0.31600624322891235, -0.3565117120742798, -0.361980676651001, -0.5285804271697998,
    -0.4974360764026642, -0.5292405486106873, -0.7103957533836365, -0.6157442927360535,
], dtype=np.float32)


def zipf_shares(num_experts: int = NUM_EXPERTS, s: float = 1.1) -> np.ndarray:
    """Target assignment share of expert e: (e+1)^-s normalised."""
    w = np.arange(1, num_experts + 1, dtype=np.float64) ** (-s)
    return w / w.sum()


# --------------------------------------------------------------------------
# bf16 and fp8 e4m3 encodings (exact, integer-only rounding)

def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (round-to-nearest-even); returns uint16 bits.
    Inputs here are finite."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    rounding = np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))
    return ((u + rounding) >> np.uint32(16)).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_e4m3_bits(v: np.ndarray) -> np.ndarray:
    """OCP fp8 e4m3 ("fn": bias 7, max 448, no inf) with round-to-nearest-
    even and saturation to +-448.  Returns uint8 codes."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    a = np.minimum(np.abs(v).astype(np.float64), FP8_E4M3_MAX)
    _, ex = np.frexp(a)                      # a = m * 2^ex, m in [0.5, 1)
    e = np.maximum(ex - 1, -6)               # unbiased exponent, subnormal floor
    step = np.ldexp(1.0, e - 3)              # spacing of representable values
    q = np.rint(a / step) * step             # exact: step is a power of two
    q = np.minimum(q, FP8_E4M3_MAX)
    _, qx = np.frexp(q)
    qe = np.where(q > 0, np.maximum(qx - 1, -6), -6)
    normal = q >= 2.0 ** -6
    mant = np.where(normal, np.rint(q / np.ldexp(1.0, qe) * 8.0) - 8.0, np.rint(q / 2.0 ** -9))
    exp_field = np.where(normal, qe + 7, 0)
    code = (exp_field.astype(np.int64) << 3) | mant.astype(np.int64)
    sign = (np.signbit(v)).astype(np.int64) << 7
    return (code | sign).astype(np.uint8)


def e4m3_bits_to_f32(c: np.ndarray) -> np.ndarray:
    c = np.ascontiguousarray(c, dtype=np.uint8).astype(np.int64)
    s = np.where((c >> 7) & 1, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.ldexp(1.0, e - 7))
    val = np.where((e == 0xF) & (m == 7), np.nan, val)
    return (s * val).astype(np.float32)


def quantise_rows_e4m3(w: np.ndarray):
    """Per-row (per output channel) symmetric e4m3 quantisation:
    scale = amax / 448 (fp32), code = e4m3(w / scale).  Returns
    (codes uint8, scales float32, dequantised float32 = fp32(code) * scale)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    amax = np.max(np.abs(w), axis=-1, keepdims=True)
    scale = (amax / np.float32(FP8_E4M3_MAX)).astype(np.float32)
    scale = np.where(scale > 0, scale, np.float32(1.0)).astype(np.float32)
    codes = f32_to_e4m3_bits((w / scale).astype(np.float32))
    deq = (e4m3_bits_to_f32(codes) * scale).astype(np.float32)
    return codes, scale[..., 0], deq


# --------------------------------------------------------------------------

@dataclass
class MoeInputs:
    """One synthetic MoE block.  ``x, gate, w1, w3, w2`` are float32 arrays of
    the exact values the device computes with; ``packed`` holds the device
    encodings (``x_bf16``, ``w1_bf16`` ... or ``w1_e4m3`` + ``w1_scale``)."""
    name: str
    T: int
    H: int
    E: int
    F: int
    dtype: str                       # "f32" | "bf16" | "fp8"
    x: np.ndarray
    gate: np.ndarray
    w1: np.ndarray
    w3: np.ndarray
    w2: np.ndarray
    packed: Dict[str, np.ndarray] = field(default_factory=dict)
    zipf: Optional[float] = None
    seed: int = 0


def make_moe_inputs(T: int, H: int = HIDDEN, E: int = NUM_EXPERTS, F: int = FFN,
                    dtype: str = "f32", zipf: Optional[float] = None,
                    seed: int = 0, name: str = "custom",
                    bias: Optional[np.ndarray] = None) -> MoeInputs:
    """Draw x ~ N(0,1) [T,H]; gate ~ N(0,0.02) [E,H]; then for each of w1, w3
    ([E,F,H]) and w2 ([E,H,F]) ~ N(0,0.02), in that order, from one PCG64
    stream.  ``dtype`` rounds x and the expert weights to bf16 ("bf16"), or
    rounds x to bf16 and quantises the expert weights to fp8 e4m3 with
    per-output-channel scales ("fp8"); the gate always stays fp32 like the
    reference router.  ``zipf`` folds the calibrated per-expert bias into
    column H-1 (see module docstring)."""
    if dtype not in ("f32", "bf16", "fp8"):
        raise ValueError(f"unknown dtype {dtype!r}")
    rng = np.random.default_rng(seed)
    std = np.float32(WEIGHT_STD)
    x = rng.standard_normal((T, H), dtype=np.float32)
    gate = rng.standard_normal((E, H), dtype=np.float32) * std
    w1 = rng.standard_normal((E, F, H), dtype=np.float32) * std
    w3 = rng.standard_normal((E, F, H), dtype=np.float32) * std
    w2 = rng.standard_normal((E, H, F), dtype=np.float32) * std
    if zipf is not None or bias is not None:
        if bias is None:
            if abs(zipf - 1.1) > 1e-12 or E != NUM_EXPERTS:
                raise ValueError("only the calibrated Zipf(1.1), 16-expert bias table exists")
            bias = ZIPF_1_1_BIAS
        x[:, H - 1] = 1.0
        gate[:, H - 1] = np.asarray(bias, dtype=np.float32)
    packed: Dict[str, np.ndarray] = {}
    if dtype in ("bf16", "fp8"):
        xb = f32_to_bf16_bits(x)
        packed["x_bf16"] = xb
        x = bf16_bits_to_f32(xb)
    if dtype == "bf16":
        for nm, w in (("w1", w1), ("w3", w3), ("w2", w2)):
            b = f32_to_bf16_bits(w)
            packed[nm + "_bf16"] = b
        w1, w3, w2 = (bf16_bits_to_f32(packed[n + "_bf16"]) for n in ("w1", "w3", "w2"))
    elif dtype == "fp8":
        deq = {}
        for nm, w in (("w1", w1), ("w3", w3), ("w2", w2)):
            codes, scale, d = quantise_rows_e4m3(w)
            packed[nm + "_e4m3"] = codes
            packed[nm + "_scale"] = scale
            deq[nm] = d
        w1, w3, w2 = deq["w1"], deq["w3"], deq["w2"]
    return MoeInputs(name=name, T=T, H=H, E=E, F=F, dtype=dtype, x=np.ascontiguousarray(x),
                     gate=np.ascontiguousarray(gate), w1=np.ascontiguousarray(w1),
                     w3=np.ascontiguousarray(w3), w2=np.ascontiguousarray(w2),
                     packed=packed, zipf=zipf, seed=seed)


# The benchmark configs that exercise the MoE block itself.
CONFIGS = {
    # C1: fp32, CPU-runnable, 512 tokens, unbiased router, seed 0.
    "c1": dict(T=512, dtype="f32", zipf=None),
    # C2: bf16 at 4096 prefill tokens (8 prompts x 512), Zipf(1.1) loads.
    "c2": dict(T=4096, dtype="bf16", zipf=1.1),
    # C5: fp8 e4m3 expert weights, bf16 activations, 8192 tokens, Zipf(1.1).
    "c5": dict(T=8192, dtype="fp8", zipf=1.1),
}


def make_config(name: str, seed: int = 0, T: Optional[int] = None) -> MoeInputs:
    cfg = dict(CONFIGS[name])
    if T is not None:
        cfg["T"] = T
    return make_moe_inputs(seed=seed, name=name, **cfg)


def c4_prompts(seed: int = 0, groups: int = 4, per_group: int = 4, prefix_len: int = 512,
               suffix_len: int = 512, vocab: int = 32064) -> list:
    """C4's prompt batch: groups x per_group prompts of prefix_len +
    suffix_len random token ids, the prompts of a group sharing their first
    prefix_len ids (default 16 prompts of 1024 ids, 4 groups sharing 512:
    16,384 token rows, 10,240 prefix-trie nodes at seed 0)."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(groups):
        pre = rng.integers(0, vocab, prefix_len)
        for _ in range(per_group):
            out.append(np.concatenate([pre, rng.integers(0, vocab, suffix_len)]).tolist())
    return out
