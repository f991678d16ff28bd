"""The allocation-free forward (aps_moe_forward_noalloc) through the C ABI:
its output equals aps_moe_forward's with a caller workspace bit for bit, on
two calls in a row with the second batch smaller than the first (the static
scratch keeps the first call's bytes), for a bf16, an fp32 and an fp8 weight
set (the fp8 one runs the folded combine and the router's x quantisation);
a batch past the scratch is refused with APS_ERR_WORKSPACE."""
import ctypes
import sys

import numpy as np
import pytest
import torch

from aps2026_amd import capi, moe, synth

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _weights(inp, dev):
    if inp.dtype == "fp8":
        codes, scales = [], []
        for nm in ("w1", "w2", "w3"):
            c = torch.from_numpy(inp.packed[nm + "_e4m3"]).to(dev)
            sc = torch.from_numpy(inp.packed[nm + "_scale"]).to(dev)
            codes.append([c[e].contiguous() for e in range(inp.E)])
            scales.append([sc[e].contiguous() for e in range(inp.E)])
        return moe.register_moe_weights_gpu(codes[0], codes[1], codes[2], compute_dtype=moe.FP8,
                                            scales=(scales[0], scales[1], scales[2]))
    lists = []
    for nm in ("w1", "w2", "w3"):
        if inp.dtype == "bf16":
            b = torch.from_numpy(inp.packed[nm + "_bf16"].view(np.int16)).to(dev).view(torch.bfloat16)
        else:
            b = torch.from_numpy(getattr(inp, nm)).to(dev)
        lists.append([b[e].contiguous() for e in range(inp.E)])
    compute = torch.bfloat16 if inp.dtype == "bf16" else torch.float32
    return moe.register_moe_weights_gpu(lists[0], lists[1], lists[2], compute_dtype=compute)


def _x(inp, dev):
    if inp.dtype in ("bf16", "fp8"):
        return torch.from_numpy(inp.packed["x_bf16"].view(np.int16)).to(dev).view(torch.bfloat16)
    return torch.from_numpy(inp.x).to(dev)


@pytest.mark.parametrize("dtype,sizes", [("bf16", (4096, 300)), ("f32", (512, 77)), ("fp8", (3000, 129))])
def test_forward_noalloc_equals_workspace_forward(gpu_device, dtype, sizes):
    L = capi.lib()
    T0 = sizes[0]
    H, F = (4096, 448)
    inp = synth.make_moe_inputs(T=T0, H=H, E=16, F=F, dtype=dtype, seed=41, name="noalloc")
    w = _weights(inp, gpu_device)
    x_all = _x(inp, gpu_device)
    gate = torch.from_numpy(inp.gate).to(gpu_device)
    code = capi.DTYPE_F32 if dtype == "f32" else capi.DTYPE_BF16   # fp8 weights take bf16 x and output
    out_dt = torch.float32 if dtype == "f32" else torch.bfloat16
    stream = ctypes.c_void_p(torch.cuda.current_stream(gpu_device).cuda_stream)
    for T in sizes:
        note(f"forward_noalloc {dtype} T={T}")
        x = x_all[:T].contiguous()
        want = moe.moe_forward_gpu(x, gate, w, out_dtype=out_dt)
        got = torch.full_like(want, float("nan"))
        rc = L.aps_moe_forward_noalloc(w.handle, ctypes.c_void_p(x.data_ptr()), code,
                                       ctypes.c_void_p(gate.data_ptr()), T, ctypes.c_void_p(got.data_ptr()),
                                       code, stream)
        assert rc == capi.APS_OK, capi.last_error()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32 if dtype == "f32" else torch.int16),
                           want.view(torch.int32 if dtype == "f32" else torch.int16))
    # past the scratch: refused before any launch
    big = L.aps_moe_noalloc_scratch_bytes() // (2 * H) + 1
    rc = L.aps_moe_forward_noalloc(w.handle, ctypes.c_void_p(x_all.data_ptr()), code,
                                   ctypes.c_void_p(gate.data_ptr()), big, ctypes.c_void_p(x_all.data_ptr()), code,
                                   stream)
    assert rc == capi.APS_ERR_WORKSPACE
    assert "static scratch" in capi.last_error()
    w.release()
