"""ctypes wrapper over the CPU oracle (liboracle_moe.so, built from
moe_oracle.c by the Makefile beside it).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker or the timed CPU
baseline, never as part of the product path.  Each function restates one
step of the reference MoE path; the reference file:line it follows is given
in moe_oracle.c.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle_moe.so")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32

_lib = None


def build() -> str:
    """Compile liboracle_moe.so with gcc (no GPU needed)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_router_logits.argtypes = [_f32p, _f32p, _i64, _i32, _i32, _f32p]
        L.oracle_quantise.argtypes = [ctypes.c_float, ctypes.c_float]
        L.oracle_quantise.restype = ctypes.c_float
        L.oracle_route_top2.argtypes = [_f32p, _i64, _i32, ctypes.c_float, ctypes.c_float, _i32p, ctypes.c_void_p]
        L.oracle_dispatch.argtypes = [_i32p, _i64, _i32, _u32p, _u32p, _u32p, _u32p]
        L.oracle_ffn_rows.argtypes = [_f32p, _i32p, _i64, _i32, _i32, _i32, _f32p, _f32p, _f32p,
                                      ctypes.c_void_p, _f32p]
        L.oracle_combine.argtypes = [_f32p, _i32p, _u32p, _i64, _i32, _f32p]
        L.oracle_moe_forward.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _i64, _i32, _i32, _i32,
                                         _f32p, ctypes.c_void_p, ctypes.c_void_p]
        L.oracle_bf16_to_f32.argtypes = [_u16p, _f32p, _i64]
        L.oracle_e4m3_to_f32.argtypes = [_u8p, _f32p, _i64]
        L.oracle_quantise_rows_e4m3.argtypes = [_f32p, _i64, _i32, _u8p, _f32p]
        L.oracle_layer_norm.argtypes = [_f32p, ctypes.c_void_p, _i64, _i32, _f32p, _f32p, ctypes.c_float,
                                        ctypes.c_void_p, _f32p, ctypes.c_void_p, ctypes.c_void_p]
        L.oracle_default_quantum.restype = ctypes.c_float
        L.oracle_linear.argtypes = [_f32p, _f32p, ctypes.c_void_p, _i64, _i32, _i32, _f32p]
        L.oracle_rope_table.argtypes = [_i64, _i32, ctypes.c_float, _f32p, _f32p]
        L.oracle_rope_tree.argtypes = [_f32p, _u32p, _i64, _i32, _i32, _f32p, _f32p]
        L.oracle_attention_tree.argtypes = [_f32p, _f32p, _f32p, _f32p, _u32p, _u32p, _i64, _i64, _i32, _i32,
                                            _i32, _i32]
        L.oracle_attention_generic.argtypes = [_f32p, _f32p, _f32p, _f32p, _u32p, _u32p, _i64, _i32, _i32, _i32,
                                               _i32]
        L.oracle_default_tie_eps.restype = ctypes.c_float
        L.oracle_num_threads.restype = ctypes.c_int
        L.oracle_set_num_threads.argtypes = [ctypes.c_int]
        _lib = L
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"oracle {what} failed with code {rc}")


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


QUANTUM = np.float32(1.0e-3)
TIE_EPS = np.float32(2.0e-2)


def num_threads() -> int:
    return lib().oracle_num_threads()


def set_num_threads(n: int) -> None:
    lib().oracle_set_num_threads(int(n))


def router_logits(x: np.ndarray, gate: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32); gate = _c(gate, np.float32)
    T, H = x.shape
    E = gate.shape[0]
    out = np.empty((T, E), np.float32)
    _check(lib().oracle_router_logits(x, gate, T, H, E, out), "router_logits")
    return out


def quantise(l: float, quantum: float = float(QUANTUM)) -> np.float32:
    return np.float32(lib().oracle_quantise(float(np.float32(l)), float(np.float32(quantum))))


def route_top2(logits: np.ndarray, quantum=QUANTUM, tie_eps=TIE_EPS) -> np.ndarray:
    """Returns routes int32 [T, 2] (slot 0 = first pick)."""
    logits = _c(logits, np.float32)
    T, E = logits.shape
    routes = np.empty((T, 2), np.int32)
    _check(lib().oracle_route_top2(logits, T, E, float(quantum), float(tie_eps), routes, None), "route_top2")
    return routes


def dispatch(routes: np.ndarray, E: int) -> Tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """Returns (counts[E], offsets[E+1], assignment_rows[2T], route_positions[2T])."""
    routes = _c(routes, np.int32)
    T = routes.shape[0]
    counts = np.empty(E, np.uint32)
    offsets = np.empty(E + 1, np.uint32)
    rows = np.empty(2 * T, np.uint32)
    pos = np.empty(2 * T, np.uint32)
    _check(lib().oracle_dispatch(routes, T, E, counts, offsets, rows, pos), "dispatch")
    return counts, offsets, rows, pos


def ffn_rows(xrows: np.ndarray, experts: np.ndarray, w1, w3, w2,
             want_act: bool = False):
    """Expert FFN for n (row, expert) pairs; returns y [n, H] (and act [n, F])."""
    xrows = _c(xrows, np.float32)
    experts = _c(experts, np.int32)
    w1 = _c(w1, np.float32); w3 = _c(w3, np.float32); w2 = _c(w2, np.float32)
    n, H = xrows.shape
    E, F, _ = w1.shape
    y = np.empty((n, H), np.float32)
    act = np.empty((n, F), np.float32) if want_act else None
    _check(lib().oracle_ffn_rows(xrows, experts, n, H, F, E, w1, w3, w2,
                                 act.ctypes.data if act is not None else None, y), "ffn_rows")
    return (y, act) if want_act else y


def combine(y: np.ndarray, routes: np.ndarray, route_positions: np.ndarray) -> np.ndarray:
    y = _c(y, np.float32)
    routes = _c(routes, np.int32)
    route_positions = _c(route_positions, np.uint32)
    T = routes.shape[0]
    H = y.shape[1]
    out = np.empty((T, H), np.float32)
    _check(lib().oracle_combine(y, routes, route_positions, T, H, out), "combine")
    return out


def moe_forward(x, gate, w1, w3, w2, want_intermediate: bool = False):
    """Whole block in the reference CPU path's order (src/layer.cu:113-148)."""
    x = _c(x, np.float32); gate = _c(gate, np.float32)
    w1 = _c(w1, np.float32); w3 = _c(w3, np.float32); w2 = _c(w2, np.float32)
    T, H = x.shape
    E, F, _ = w1.shape
    out = np.empty((T, H), np.float32)
    logits = np.empty((T, E), np.float32) if want_intermediate else None
    routes = np.empty((T, 2), np.int32) if want_intermediate else None
    _check(lib().oracle_moe_forward(x, gate, w1, w3, w2, T, H, F, E, out,
                                    logits.ctypes.data if logits is not None else None,
                                    routes.ctypes.data if routes is not None else None), "moe_forward")
    return (out, logits, routes) if want_intermediate else out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    bits = _c(bits, np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().oracle_bf16_to_f32(bits.reshape(-1), out.reshape(-1), bits.size)
    return out


def e4m3_to_f32(codes: np.ndarray) -> np.ndarray:
    codes = _c(codes, np.uint8)
    out = np.empty(codes.shape, np.float32)
    lib().oracle_e4m3_to_f32(codes.reshape(-1), out.reshape(-1), codes.size)
    return out


def round_to_bf16(v: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 value (ties to even), as float32; finite
    inputs."""
    u = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def quantise_rows_e4m3(rows: np.ndarray):
    """Per-row e4m3: (codes uint8, scale float32 per row); scale = amax/448."""
    rows = _c(rows, np.float32)
    r, n = rows.shape
    codes = np.empty((r, n), np.uint8)
    scale = np.empty(r, np.float32)
    lib().oracle_quantise_rows_e4m3(rows, r, n, codes, scale)
    return codes, scale


def dequantise_rows_e4m3(codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    return (e4m3_to_f32(codes) * np.asarray(scale, np.float32)[:, None]).astype(np.float32)


def fp8_ffn_rows(x_rows: np.ndarray, experts: np.ndarray, w1, w3, w2):
    """The fp8 path's expert FFN for n (row, expert) pairs (config C5, fp8 experts):
    x rows quantised per row to e4m3, the dequantised values through the
    gate/up GEMMs and SiLU (fp32), the activations rounded to bf16 and
    quantised per row to e4m3, then the w2 GEMM on their dequantised values.
    w1/w3/w2 are the dequantised weights (codes x per-channel scales).
    Returns (y [n, H] float32, act_bf16 [n, F] float32)."""
    xq, xs = quantise_rows_e4m3(x_rows)
    xh = dequantise_rows_e4m3(xq, xs)
    _, act = ffn_rows(xh, experts, w1, w3, w2, want_act=True)
    act_b = round_to_bf16(act)
    aq, as_ = quantise_rows_e4m3(act_b)
    ah = dequantise_rows_e4m3(aq, as_).astype(np.float64)
    w2 = np.asarray(w2, np.float32)
    y = np.empty((x_rows.shape[0], w2.shape[1]), np.float32)
    for e in np.unique(experts):
        idx = np.where(experts == e)[0]
        y[idx] = (ah[idx] @ w2[e].astype(np.float64).T).astype(np.float32)
    return y, act_b


def reference_path(x, gate, w1, w3, w2):
    """Full staged oracle (GPU-path semantics): returns a dict with logits,
    routes, counts, offsets, assignment_rows, route_positions, y, out."""
    logits = router_logits(x, gate)
    routes = route_top2(logits)
    E = gate.shape[0]
    counts, offsets, rows, pos = dispatch(routes, E)
    experts = np.repeat(np.arange(E, dtype=np.int32), counts.astype(np.int64))
    y = ffn_rows(np.asarray(x)[rows.astype(np.int64)], experts, w1, w3, w2)
    out = combine(y, routes, pos)
    return dict(logits=logits, routes=routes, counts=counts, offsets=offsets,
                assignment_rows=rows, route_positions=pos, y=y, out=out)


def layer_norm(x: np.ndarray, weight: np.ndarray, bias: np.ndarray, eps: float = 1e-5,
               residual: Optional[np.ndarray] = None):
    """The decoder layer's LayerNorm with the reference GPU kernels' operation
    order (moe_oracle.c, oracle_layer_norm).  With ``residual`` it is
    add_layer_norm: v = x + residual.  Returns (y, v, mean, inv), all float32."""
    x = _c(x, np.float32)
    rows, h = x.shape
    w = _c(weight, np.float32)
    b = _c(bias, np.float32)
    res = None if residual is None else _c(residual, np.float32)
    if res is not None and res.shape != x.shape:
        raise ValueError("add layer norm shape")
    if w.shape != (h,) or b.shape != (h,):
        raise ValueError("layer norm shape")
    y = np.empty_like(x)
    v = np.empty_like(x)
    mean = np.empty(rows, np.float32)
    inv = np.empty(rows, np.float32)
    lib().oracle_layer_norm(x, None if res is None else res.ctypes.data, rows, h, w, b, np.float32(eps),
                            v.ctypes.data, y, mean.ctypes.data, inv.ctypes.data)
    return y, v, mean, inv


def prefix_dedup(input_ids, vocab_size: int = 32064, max_positions: int = 4096):
    """Prefix trie of a prompt batch, pure Python (small and medium batches).

    Restates PhiTinyMoEModel::generate (reference src/model.cu:44-117):
    lengths checked first over the whole batch ("empty input", "sequence is
    too long"), then one walk sequence by sequence with a dict from (parent,
    token) to child; a new child gets the next node id and records its token,
    depth and ancestor chain root .. node; "token out of vocabulary" is
    raised at the first bad token of the walk.  An empty batch raises
    RuntimeError("generate received an empty input batch") (src/model.cu:47-49).
    Returns (token_node, node_token, node_depth, node_anc) as lists; node_anc
    holds the chains without padding."""
    if len(input_ids) == 0:
        raise RuntimeError("generate received an empty input batch")
    for seq in input_ids:
        if len(seq) == 0:
            raise ValueError("empty input")
        if len(seq) > max_positions:
            raise ValueError("sequence is too long")
    children = {}
    token_node, node_token, node_depth, node_anc = [], [], [], []
    for seq in input_ids:
        parent = -1
        chain = []
        for si, tok in enumerate(seq):
            tok = int(tok)
            if tok < 0 or tok >= vocab_size:
                raise ValueError("token out of vocabulary")
            key = (parent, tok)
            node = children.get(key)
            if node is None:
                node = len(node_token)
                children[key] = node
                node_token.append(tok)
                node_depth.append(si)
                node_anc.append(chain + [node])
            chain.append(node)  # chain = nodes of positions 0 .. si of this sequence
            token_node.append(node)
            parent = node
    return token_node, node_token, node_depth, node_anc


def gather_rows(x: np.ndarray, rows) -> np.ndarray:
    """out[i] = x[rows[i]] (reference k_gather_rows, src/tensor.cu:2635-2642)."""
    return np.ascontiguousarray(x[np.asarray(rows, dtype=np.int64)])


def model_bin_index(data: bytes):
    """The index of a model.bin image, pure Python (reference
    src/model_loader.cu:14-31): u32 count, then per entry u32 name_len, the
    name, u32 ndim, ndim u32 dims, u64 offset, u64 bytes, little-endian.
    Returns {name: (shape, offset, bytes)} (first entry of a name wins);
    raises RuntimeError("truncated model.bin") when the index runs past the
    end."""
    import struct
    pos = 0

    def take(fmt):
        nonlocal pos
        n = struct.calcsize(fmt)
        if pos + n > len(data):
            raise RuntimeError("truncated model.bin")
        v = struct.unpack_from(fmt, data, pos)
        pos += n
        return v

    (count,) = take("<I")
    out = {}
    for _ in range(count):
        (name_len,) = take("<I")
        if pos + name_len > len(data):
            raise RuntimeError("truncated model.bin")
        name = data[pos:pos + name_len].decode("utf-8", "surrogateescape")
        pos += name_len
        (ndim,) = take("<I")
        shape = take(f"<{ndim}I") if ndim else ()
        offset, nbytes = take("<QQ")
        out.setdefault(name, (tuple(shape), offset, nbytes))
    return out


def bf16_split(v: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """hi = bf16(v), lo = bf16(v - hi), round to nearest even, as fp32 arrays
    (reference k_pack_bf16_weight and the split in
    k_matmul_transposed_bf16_wmma, src/tensor.cu:141-145, 537-540)."""
    def rn(a):
        u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
        return r.view(np.float32)
    v = np.ascontiguousarray(v, np.float32)
    hi = rn(v)
    lo = rn((v - hi).astype(np.float32))   # v - hi is exact in fp32
    return hi, lo


def linear_split_bf16(x: np.ndarray, w: np.ndarray, bias: Optional[np.ndarray] = None,
                      all_terms: bool = False) -> np.ndarray:
    """The reference's USE_TC Linear (src/tensor.cu:514-584, 3042-3055,
    3121-3142): sum over k of x_hi w_hi + x_hi w_lo + x_lo w_hi (+ x_lo w_lo
    under USE_TC_ALL), then + bias.  The tensor cores' accumulation order is
    not specified, so this restatement sums the exact bf16 products in fp64
    and rounds once: the value every fp32 accumulation order approximates."""
    xh, xl = bf16_split(x)
    wh, wl = bf16_split(w)
    xh, xl, wh, wl = (a.astype(np.float64) for a in (xh, xl, wh, wl))
    y = xh @ wh.T + xh @ wl.T + xl @ wh.T
    if all_terms:
        y += xl @ wl.T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return y.astype(np.float32)


SLIDING_WINDOW = 2047   # reference include/config.h:17
ROPE_THETA = 10000.0    # reference include/config.h:18


def linear(x: np.ndarray, w: np.ndarray, bias: Optional[np.ndarray] = None) -> np.ndarray:
    """y = x w^T (+ bias): one fp32 FMA chain over k ascending per output,
    the bias added once (reference k_matmul_transposed_8x8 and its epilogue,
    src/tensor.cu:715-800)."""
    x = _c(x, np.float32); w = _c(w, np.float32)
    T, K = x.shape
    N = w.shape[0]
    y = np.empty((T, N), np.float32)
    b = _c(bias, np.float32) if bias is not None else None
    _check(lib().oracle_linear(x, w, b.ctypes.data_as(ctypes.c_void_p) if b is not None else None, T, K, N, y),
           "linear")
    return y


def rope_table(max_seq: int, head_dim: int, theta: float = ROPE_THETA):
    """(cos, sin) [max_seq, head_dim / 2] fp32 (reference src/tensor.cu:2703-2735)."""
    half = head_dim // 2
    c = np.empty((max_seq, half), np.float32)
    sn = np.empty((max_seq, half), np.float32)
    lib().oracle_rope_table(max_seq, head_dim, theta, c, sn)
    return c, sn


def rope_tree(x: np.ndarray, row_pos, heads: int, head_dim: int, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """RoPE of x [rows, heads * head_dim] at each row's position (reference
    k_rope, src/tensor.cu:2180-2197); returns a new array."""
    y = _c(x, np.float32).copy()
    pos = _c(row_pos, np.uint32)
    lib().oracle_rope_tree(y, pos, pos.shape[0], heads, head_dim, _c(cos, np.float32), _c(sin, np.float32))
    return y


def attention_generic(q, k, v, seg_offset, seg_pos, q_heads: int, kv_heads: int, head_dim: int,
                      window_max: int = SLIDING_WINDOW) -> np.ndarray:
    """Packed-sequence attention for head layouts other than GQA-4 (reference
    k_attention, src/tensor.cu:2209-2274); out [rows, q_heads * head_dim]."""
    pos = _c(seg_pos, np.uint32)
    rows = pos.shape[0]
    out = np.empty((rows, q_heads * head_dim), np.float32)
    lib().oracle_attention_generic(_c(q, np.float32), _c(k, np.float32), _c(v, np.float32), out,
                                   _c(seg_offset, np.uint32), pos, rows, q_heads, kv_heads, head_dim, window_max)
    return out


def attention_tree(q, k, v, row_pos, anc, anc_stride: int, q_heads: int, kv_heads: int, head_dim: int,
                   window_max: int = SLIDING_WINDOW) -> np.ndarray:
    """GQA tree attention over ancestor chains (reference
    k_attention_tree_gqa4, src/tensor.cu:2407-2633); out [rows, q_heads * head_dim]."""
    pos = _c(row_pos, np.uint32)
    rows = pos.shape[0]
    out = np.empty((rows, q_heads * head_dim), np.float32)
    lib().oracle_attention_tree(_c(q, np.float32), _c(k, np.float32), _c(v, np.float32), out, pos,
                                _c(anc, np.uint32), anc_stride, rows, q_heads, kv_heads, head_dim, window_max)
    return out
