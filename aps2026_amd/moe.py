"""Host-side mirror of the reference operator API for the MoE feed-forward
path, over the C ABI (include/aps_moe.h).  PyTorch supplies device memory and
the current HIP stream; every computation runs in the HIP kernels of
libaps_moe.so.

Reference API mirrored (file:line in the reference tree):
  tensor_ops::matmul_transposed_gpu      include/tensor.h:72 (router path)
  tensor_ops::register_moe_weights_gpu   include/tensor.h:142-145
  tensor_ops::moe_forward_grouped_gpu    include/tensor.h:146-147
  PhiMLP / PhiMoE                        include/layer.h:23-43

As in the reference, shape and handle errors raise ``ValueError`` (the
reference's std::invalid_argument) and runtime failures ``RuntimeError``.
There is no CPU execution path: ``use_gpu=False`` raises, because the only
CPU implementation in this repository is the test oracle.
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Sequence

import torch

from . import capi
from .capi import ApsError

_DTYPE_CODE = {torch.float32: capi.DTYPE_F32, torch.bfloat16: capi.DTYPE_BF16,
               torch.float8_e4m3fn: capi.DTYPE_E4M3, torch.uint8: capi.DTYPE_E4M3}
FP8 = torch.float8_e4m3fn


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: Optional[torch.Tensor]) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _raise(e: ApsError):
    if e.code in (capi.APS_ERR_SHAPE, capi.APS_ERR_HANDLE, capi.APS_ERR_DTYPE,
                  capi.APS_ERR_ARG, capi.APS_ERR_WORKSPACE):
        raise ValueError(e.message) from None
    raise RuntimeError(e.message) from None


def _call(rc: int) -> None:
    try:
        capi.check(rc)
    except ApsError as e:
        _raise(e)


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


class MoeWeights:
    """A registered expert weight set (the reference's 1-based handle)."""

    def __init__(self, w1: Sequence[torch.Tensor], w2: Sequence[torch.Tensor],
                 w3: Sequence[torch.Tensor], compute_dtype: torch.dtype = torch.bfloat16,
                 scales: Optional[tuple] = None):
        """fp8 (compute_dtype torch.float8_e4m3fn): w1/w2/w3 hold e4m3 codes
        (uint8 or float8_e4m3fn tensors) and ``scales = (s1, s2, s3)`` the
        per-output-channel fp32 scales ([F], [H], [F] per expert)."""
        E = len(w1)
        _require(len(w2) == E and len(w3) == E, "MoE weight table size")
        _require(E >= 1, "MoE weight table size")
        F, H = w1[0].shape
        src = w1[0].dtype
        for t, shp in [(t, (F, H)) for t in list(w1) + list(w3)] + [(t, (H, F)) for t in w2]:
            _require(tuple(t.shape) == shp and t.dtype == src and t.is_cuda and t.is_contiguous(),
                     "MoE weight table size")
        _require(src in _DTYPE_CODE, f"unsupported weight dtype {src}")
        _require(compute_dtype in _DTYPE_CODE, f"unsupported compute dtype {compute_dtype}")
        self.num_experts, self.hidden, self.ffn = E, H, F
        self.compute_dtype = compute_dtype
        self.device = w1[0].device
        arr = ctypes.c_void_p * E
        self._keep = [arr(*[t.data_ptr() for t in w1]), arr(*[t.data_ptr() for t in w3]),
                      arr(*[t.data_ptr() for t in w2])]
        sc = [None, None, None]
        if compute_dtype == FP8:
            _require(scales is not None and len(scales) == 3, "fp8 weights need (s1, s2, s3) scale tables")
            s1, s2, s3 = scales
            for lst, n in ((s1, F), (s3, F), (s2, H)):
                _require(len(lst) == E and all(t.dtype == torch.float32 and t.numel() == n and t.is_cuda
                                               and t.is_contiguous() for t in lst), "MoE weight table size")
            fa = ctypes.c_void_p * E
            self._keep += [fa(*[t.data_ptr() for t in s1]), fa(*[t.data_ptr() for t in s3]),
                           fa(*[t.data_ptr() for t in s2])]
            sc = [ctypes.cast(k, ctypes.POINTER(ctypes.c_void_p)) for k in self._keep[3:]]
        desc = capi.WeightsDesc(E, H, F, _DTYPE_CODE[src], _DTYPE_CODE[compute_dtype],
                                ctypes.cast(self._keep[0], ctypes.POINTER(ctypes.c_void_p)),
                                ctypes.cast(self._keep[1], ctypes.POINTER(ctypes.c_void_p)),
                                ctypes.cast(self._keep[2], ctypes.POINTER(ctypes.c_void_p)),
                                sc[0], sc[1], sc[2])
        h = ctypes.c_uint64(0)
        with torch.cuda.device(self.device):
            _call(capi.lib().aps_moe_weights_register(ctypes.byref(desc), _stream(self.device), ctypes.byref(h)))
        self.handle = h.value
        self._ws: Optional[torch.Tensor] = None

    @property
    def x_dtype(self) -> torch.dtype:
        return torch.float32 if self.compute_dtype == torch.float32 else torch.bfloat16

    def layout(self, rows: int) -> capi.WsLayout:
        L = capi.WsLayout()
        _call(capi.lib().aps_moe_workspace_layout(self.handle, rows, ctypes.byref(L)))
        return L

    def workspace(self, rows: int):
        """Grow-only device workspace (the reference's moe_scratch,
        src/tensor.cu:1227-1291).  Calls sharing it must be stream-ordered."""
        L = self.layout(rows)
        if self._ws is None or self._ws.numel() < L.total_bytes:
            self._ws = torch.empty(max(L.total_bytes, 1), dtype=torch.uint8, device=self.device)
        return self._ws, L

    def release(self) -> None:
        if self.handle:
            _call(capi.lib().aps_moe_weights_release(self.handle))
            self.handle = 0

    def plan_views(self, rows: int) -> Dict[str, torch.Tensor]:
        """Views of the routing plan and intermediates left in the workspace
        by the last forward call with `rows` tokens."""
        ws, L = self.workspace(rows)
        E, H, F = self.num_experts, self.hidden, self.ffn
        elt = torch.float32 if self.compute_dtype == torch.float32 else torch.bfloat16

        def view(off, n, dt, shape):
            nbytes = n * torch.empty((), dtype=dt).element_size()
            return ws[off:off + nbytes].view(dt).view(*shape)

        A = 2 * rows
        d = dict(
            logits=view(L.logits, rows * E, torch.float32, (rows, E)),
            routes=view(L.routes, A, torch.uint8, (rows, 2)),
            counts=view(L.counts, E, torch.int32, (E,)),
            offsets=view(L.offsets, E + 1, torch.int32, (E + 1,)),
            assignment_rows=view(L.assignment_rows, A, torch.int32, (A,)),
            route_positions=view(L.route_positions, A, torch.int32, (A,)),
            act=view(L.act, A * F, elt, (A, F)),
            y=view(L.y, A * H, elt, (A, H)),
        )
        if self.compute_dtype == FP8:
            kp = (F + 127) // 128 * 128
            d.update(xq=view(L.xq, rows * H, torch.uint8, (rows, H)),
                     x_scale=view(L.xq_scale, rows, torch.float32, (rows,)),
                     actq=view(L.actq, A * kp, torch.uint8, (A, kp)),
                     act_scale=view(L.act_scale, A, torch.float32, (A,)))
        return d


def register_moe_weights_gpu(w1: Sequence[torch.Tensor], w2: Sequence[torch.Tensor],
                             w3: Sequence[torch.Tensor],
                             compute_dtype: torch.dtype = torch.bfloat16,
                             scales: Optional[tuple] = None) -> MoeWeights:
    """reference include/tensor.h:142-145 (argument order w1, w2, w3);
    ``scales`` = (s1, s2, s3) per-channel tables for fp8 weights."""
    return MoeWeights(w1, w2, w3, compute_dtype, scales)


def matmul_transposed_gpu(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
    """c[m, n] = a[m, k] . b[n, k]^T for the router shape (n = experts <= 64,
    fp32 b, one FMA chain per output, k ascending).  reference
    include/tensor.h:72 on its narrow path (src/tensor.cu:3058-3061)."""
    _require(a.dim() == 2 and b.dim() == 2 and c.dim() == 2, "matmul_transposed_gpu shape")
    m, k = a.shape
    n = b.shape[0]
    _require(b.shape[1] == k and tuple(c.shape) == (m, n), "matmul_transposed_gpu shape")
    _require(b.dtype == torch.float32 and c.dtype == torch.float32 and a.dtype in _DTYPE_CODE,
             "matmul_transposed_gpu dtype")
    _require(a.is_contiguous() and b.is_contiguous() and c.is_contiguous(), "matmul_transposed_gpu layout")
    _call(capi.lib().aps_router_logits(_ptr(a), _DTYPE_CODE[a.dtype], _ptr(b), m, k, n, _ptr(c),
                                       _stream(a.device)))
    return c


NORM_EPS = 1.0e-5  # reference include/config.h:19


def _check_ln(x, weight, bias, y, what, residual=None):
    _require(x.dim() >= 1 and x.dtype == torch.float32 and x.is_contiguous(), f"{what} shape")
    h = x.shape[-1]
    for t in (weight, bias):
        _require(t.dtype == torch.float32 and t.is_contiguous() and t.numel() == h, f"{what} shape")
    _require(y.dtype == torch.float32 and y.is_contiguous() and y.numel() == x.numel(), f"{what} shape")
    if residual is not None:
        _require(residual.dtype == torch.float32 and residual.is_contiguous() and residual.numel() == x.numel(),
                 f"{what} shape")
    return x.numel() // h, h


def layer_norm_gpu(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float, y: torch.Tensor):
    """y = LayerNorm(x) over the last dimension with the reference GPU kernel's
    arithmetic (serial ascending sums, fused variance chain).  reference
    include/tensor.h:86-87, src/tensor.cu:3262-3280."""
    rows, h = _check_ln(x, weight, bias, y, "layer norm")
    _call(capi.lib().aps_layer_norm(_ptr(x), _ptr(weight), _ptr(bias), rows, h, eps, _ptr(y), _stream(x.device)))
    return y


def add_layer_norm_gpu(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                       eps: float, y: torch.Tensor):
    """x += residual in place, then y = LayerNorm(x).  reference
    include/tensor.h:88-90, src/tensor.cu:3282-3295."""
    rows, h = _check_ln(x, weight, bias, y, "add layer norm", residual)
    _call(capi.lib().aps_add_layer_norm(_ptr(x), _ptr(residual), _ptr(weight), _ptr(bias), rows, h, eps, _ptr(y),
                                        _stream(x.device)))
    return y


def _check_x(x: torch.Tensor, w: MoeWeights, allow_f32: bool = False):
    """allow_f32: the fused entry points also take fp32 x with a bf16 weight
    set (the reference's activations are fp32); the FFN then reads a bf16 copy."""
    _require(x.dim() == 2 and x.shape[1] == w.hidden and x.is_contiguous() and x.is_cuda,
             "grouped MoE shape or handle")
    ok = x.dtype == w.x_dtype or (allow_f32 and x.dtype == torch.float32 and w.compute_dtype == torch.bfloat16)
    _require(ok, f"x must be {w.x_dtype} for this weight set")


def _out(x: torch.Tensor, w: MoeWeights, out: Optional[torch.Tensor], out_dtype: Optional[torch.dtype]):
    if out is None:
        out = torch.empty((x.shape[0], w.hidden), dtype=out_dtype or x.dtype, device=x.device)
    _require(tuple(out.shape) == (x.shape[0], w.hidden) and out.is_contiguous() and out.dtype in _DTYPE_CODE,
             "grouped MoE shape or handle")
    return out


def moe_forward_grouped_gpu(x: torch.Tensor, router: torch.Tensor, weights: MoeWeights,
                            out: Optional[torch.Tensor] = None,
                            out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """reference include/tensor.h:146-147: routing from precomputed router
    logits [rows, E], then dispatch, grouped expert FFN and combine."""
    _check_x(x, weights, allow_f32=True)
    rows = x.shape[0]
    _require(router.dim() == 2 and tuple(router.shape) == (rows, weights.num_experts) and
             router.dtype == torch.float32 and router.is_contiguous(), "grouped MoE shape or handle")
    out = _out(x, weights, out, out_dtype)
    ws, L = weights.workspace(rows)
    _call(capi.lib().aps_moe_forward_grouped(weights.handle, _ptr(x), _DTYPE_CODE[x.dtype], _ptr(router),
                                             rows, _ptr(out), _DTYPE_CODE[out.dtype], _ptr(ws),
                                             ws.numel(), _stream(x.device)))
    return out


def moe_forward_gpu(x: torch.Tensor, gate: torch.Tensor, weights: MoeWeights,
                    out: Optional[torch.Tensor] = None,
                    out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Router GEMM + grouped path in one call (the GPU branch of
    PhiMoE::forward, reference src/layer.cu:113-121)."""
    _check_x(x, weights, allow_f32=True)
    _require(tuple(gate.shape) == (weights.num_experts, weights.hidden) and gate.dtype == torch.float32
             and gate.is_contiguous(), "router gate shape")
    out = _out(x, weights, out, out_dtype)
    ws, L = weights.workspace(x.shape[0])
    _call(capi.lib().aps_moe_forward(weights.handle, _ptr(x), _DTYPE_CODE[x.dtype], _ptr(gate), x.shape[0],
                                     _ptr(out), _DTYPE_CODE[out.dtype], _ptr(ws), ws.numel(),
                                     _stream(x.device)))
    return out


# ---- individual stages -----------------------------------------------------

def route_top2(logits: torch.Tensor) -> torch.Tensor:
    """Quantised greedy top-2 (reference k_moe_top2); returns u8 [rows, 2]."""
    rows, E = logits.shape
    routes = torch.empty((rows, 2), dtype=torch.uint8, device=logits.device)
    _call(capi.lib().aps_moe_route_top2(_ptr(logits), rows, E, _ptr(routes), _stream(logits.device)))
    return routes


def dispatch(routes: torch.Tensor, num_experts: int, check_ids: bool = True):
    """Stable counting-sort dispatch; returns (counts, offsets,
    assignment_rows, route_positions) as int32 tensors (u32 values).
    Route ids >= num_experts are clamped by the kernels (every index stays in
    range) and counted; with check_ids (the default) the call waits for the
    count and raises ValueError when it is not zero."""
    rows = routes.shape[0]
    dev = routes.device
    counts = torch.empty(num_experts, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    arows = torch.empty(max(2 * rows, 1), dtype=torch.int32, device=dev)[:2 * rows]
    rpos = torch.empty(max(2 * rows, 1), dtype=torch.int32, device=dev)[:2 * rows]
    nbytes = capi.lib().aps_moe_dispatch_workspace_size(rows, num_experts)
    scratch = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    _call(capi.lib().aps_moe_dispatch(_ptr(routes), rows, num_experts, _ptr(counts), _ptr(offsets),
                                      _ptr(arows), _ptr(rpos), _ptr(scratch), nbytes, _stream(dev)))
    if check_ids:
        bad = int(scratch[nbytes - 4:nbytes].view(torch.int32).item())
        if bad:
            raise ValueError(f"dispatch: {bad} route ids >= num_experts ({num_experts})")
    return counts, offsets, arows, rpos


def expert_ffn(weights: MoeWeights, x: torch.Tensor, offsets: torch.Tensor,
               assignment_rows: torch.Tensor) -> torch.Tensor:
    """Grouped expert FFN over permuted assignments; returns y_perm [2*rows, H]."""
    _check_x(x, weights)
    rows = x.shape[0]
    elt = weights.x_dtype
    act = torch.empty((max(2 * rows, 1), weights.ffn), dtype=elt, device=x.device)
    y = torch.empty((max(2 * rows, 1), weights.hidden), dtype=elt, device=x.device)
    _call(capi.lib().aps_moe_expert_ffn(weights.handle, _ptr(x), _DTYPE_CODE[x.dtype], rows, _ptr(offsets),
                                        _ptr(assignment_rows), _ptr(act), None, _ptr(y), _stream(x.device)))
    return y[:2 * rows]


def combine(y_perm: torch.Tensor, route_positions: torch.Tensor, rows: int,
            out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    H = y_perm.shape[1]
    out = torch.empty((rows, H), dtype=out_dtype, device=y_perm.device)
    _call(capi.lib().aps_moe_combine(_ptr(y_perm), _DTYPE_CODE[y_perm.dtype], _ptr(route_positions), rows, H,
                                     _ptr(out), _DTYPE_CODE[out_dtype], _stream(y_perm.device)))
    return out


# ---- layer classes (reference include/layer.h:23-43) -----------------------

class PhiMLP:
    """One expert: w1, w3 [F, H], w2 [H, F] (reference include/layer.h:23-32)."""

    def __init__(self, w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor):
        self._w1, self._w2, self._w3 = w1, w2, w3

    def w1(self) -> torch.Tensor:
        return self._w1

    def w2(self) -> torch.Tensor:
        return self._w2

    def w3(self) -> torch.Tensor:
        return self._w3


class PhiMoE:
    """Router + experts (reference include/layer.h:34-43).  Built from
    tensors instead of a ModelLoader; registers the expert weights once, like
    the reference constructor (src/layer.cu:94-111)."""

    def __init__(self, gate: torch.Tensor, experts: List[PhiMLP],
                 compute_dtype: torch.dtype = torch.bfloat16):
        self.gate_ = gate.contiguous().to(torch.float32)
        self.experts_ = experts
        self.weights = register_moe_weights_gpu([e.w1() for e in experts], [e.w2() for e in experts],
                                                [e.w3() for e in experts], compute_dtype)
        self.gpu_weights_handle_ = self.weights.handle

    def forward(self, x: torch.Tensor, use_gpu: bool = True,
                out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        if not use_gpu:
            raise RuntimeError("PhiMoE.forward: this build has no CPU execution path (use_gpu=False)")
        return moe_forward_gpu(x, self.gate_, self.weights, out_dtype=out_dtype)

    def route(self, logits: torch.Tensor) -> torch.Tensor:
        """Per-token (first, second) expert ids (reference PhiMoE::route)."""
        return route_top2(logits)
