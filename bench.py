"""Benchmark of the MoE feed-forward block on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2]

`--config c3` times one whole decoder layer (input LayerNorm, fp32 q/k/v
projections, RoPE, tree attention, o projection, residual add+LayerNorm, bf16
MoE block) on the 4096 prefix-trie rows of 8 prompts x 512 ids, chaining
forward_carry through 4 random-init layers.  `--config c4` times the whole
32-layer model's prefill (generate) on C4's 16 prompts x 1024 ids: host
prefix trie, 10,240 node rows through 32 layers, final norm, last rows, LM
head; its value counts prompt tokens.  Both report one layer's stages.
`--config load` times reading one MoE layer from a model.bin into HBM.

One step = one full MoE block (router GEMM, quantised top-2, dispatch,
grouped w1||w3 + SwiGLU, grouped w2, combine) over one batch of synthetic
tokens already resident in HBM.  Workload (default): benchmark config C2 --
4096 tokens, hidden 4096, 16 experts top-2, expert FFN 448, bf16, router bias
giving Zipf(1.1) expert loads.  Steps rotate over LAYERS distinct device
copies of the expert weights (4 x 176 MB > the 256 MB MALL), as consecutive
decoder layers would, so expert weights stream from HBM every step instead
of sitting in the Infinity Cache.

Timing: untimed steps run for --settle seconds (default 0.5) and then W
warm-up steps, so that the K timed steps see the clocks of sustained work
(from idle the first tens of milliseconds run slower); the timed region is
bracketed by device synchronisation.

Prints ONE JSON line.  `roofline` covers the dominant kernel (the grouped
w1||w3 + SwiGLU GEMM, k_ffn_up<Bf16Fmt>, or k_ffn_up<Fp8Fmt> for --config c5),
timed with HIP events on the stream it is launched on; its `traffic` is the
HBM bytes per launch measured with rocprofv3 counters (TRAFFIC_KIB below).
`cpu_baseline` times the CPU oracle (the reference CPU-path algorithm,
src/layer.cu:113-148) on the host cores for about --cpu-seconds.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-block prefill tokens/s + grouped-GEMM % MFMA peak, 4096 tok, 1 GPU"
PEAK_BF16 = 2.5e15       # MI355X dense bf16 MFMA, FLOP/s
PEAK_FP8 = 5.0e15        # MI355X dense fp8 MFMA, FLOP/s
PEAK_F32 = 157.3e12
PEAK_HBM = 8.0e12        # bytes/s
LAYERS = 4
COPY_PROBE_BYTES = 256 << 20
# HBM bytes per launch of the roofline kernel, from two rocprofv3 counter runs
# (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch, of `bench.py --config C
# --steps 3 --warmup 1 --cpu-baseline skip --copy-probe`), each scaled by what
# the counter reads for the 256 MiB copy probe: FETCH_SIZE 131089.0 KiB
# (x 1.9997), WRITE_SIZE 262144 KiB (x 1.0).  Summary and commands:
# profiles/moe_forward_hbm_traffic.md.  Re-measure when a GEMM kernel changes.
TRAFFIC_KIB = {"c2": (116953.7, 7168.0), "c5": (95038.3, 14336.0)}
FETCH_SCALE, WRITE_SCALE = 262144.0 / 131089.0, 1.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default 200; 20 for --config c3, 3 for c4)")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--settle", type=float, default=0.5,
                    help="seconds of untimed steps before the warm-up steps: the GPU raises its clocks over the "
                         "first tens of milliseconds of sustained work (5 warm-up + 50 timed steps from idle "
                         "read about 16%% slower than the steady state)")
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5", "load"])
    ap.add_argument("--proj", default="fp32", choices=["fp32", "tc", "tc_all"],
                    help="c3 / c4 attention projections: fp32 FMA chains (the reference's default build, bit-exact), "
                         "or the reference's optional split-bf16 tensor-core Linear: tc = three products (USE_TC; "
                         "at c4 the LM head and layer 31 as the reference selects), tc_all = four products on every "
                         "layer (USE_TC_ALL)")
    ap.add_argument("--host", default="py", choices=["py", "cpp"],
                    help="c4: drive the prefill through the Python mirror (aps2026_amd/decoder.py) or the C++ "
                         "drop-in PhiTinyMoEModel::generate (include/model.h, through tests/cpp/libmodel_drive.so)")
    ap.add_argument("--cpu-baseline", default="auto", choices=["auto", "skip"])
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="CPU baseline: repeat full-batch runs until this much time is spent (at least 2 runs)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="run one 256 MiB device-to-device copy before the steps (scale reference for the "
                         "FETCH_SIZE / WRITE_SIZE counter passes)")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = {"c3": 20, "c4": 3}.get(args.config, 200)
    return args


def load_bench(args):
    """--config load: one full-size MoE layer (gate + 16 experts, fp32, 352 MB)
    written to a model.bin in the temp directory, then, per step, the
    reference's load sequence: ModelLoader index parse, every tensor to HBM
    (ModelLoader.load_all: file reads into two pinned staging buffers
    overlapped with the uploads), and registration (bf16 tile packing).  The file is read from the page cache after the first step."""
    import tempfile

    import torch
    from aps2026_amd import moe
    from aps2026_amd.model_loader import ModelLoader, moe_layer_tensors, write_model_bin

    dev = torch.device("cuda:0")
    H, E, F = 4096, 16, 448
    rng = np.random.default_rng(0)
    tensors = moe_layer_tensors(0, (0.02 * rng.standard_normal((E, H))).astype(np.float32),
                                [(0.02 * rng.standard_normal((F, H))).astype(np.float32) for _ in range(E)],
                                [(0.02 * rng.standard_normal((H, F))).astype(np.float32) for _ in range(E)],
                                [(0.02 * rng.standard_normal((F, H))).astype(np.float32) for _ in range(E)])
    nbytes = sum(t.nbytes for t in tensors.values())
    fd, path = tempfile.mkstemp(suffix=".bin")
    os.close(fd)
    try:
        write_model_bin(path, tensors)
        del tensors
        base = "model.layers.0.block_sparse_moe"

        def step():
            t0 = time.perf_counter()
            m = ModelLoader(path)
            names = [f"{base}.gate.weight"] + [f"{base}.experts.{e}.{nm}.weight"
                                               for nm in ("w1", "w2", "w3") for e in range(E)]
            got = m.load_all(names, dev)
            gate, ws = got[0], [got[1 + k * E:1 + (k + 1) * E] for k in range(3)]
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            w = moe.register_moe_weights_gpu(*ws, compute_dtype=torch.bfloat16)
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            w.release()
            del gate, ws
            return t1 - t0, t2 - t1

        step()  # page cache and allocator warm-up
        n = max(1, min(args.steps, 5))
        runs = [step() for _ in range(n)]
        # achievable pinned host -> device rate of this box, for scale
        src = torch.empty(256 << 20, dtype=torch.uint8, pin_memory=True)
        dst = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst.copy_(src)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        h2d = 4 * (256 << 20) / (time.perf_counter() - t0)
    finally:
        os.unlink(path)
    load_s = statistics.median(r[0] for r in runs)
    reg_s = statistics.median(r[1] for r in runs)
    value = nbytes / load_s
    print(json.dumps({
        "metric": "model.bin MoE layer load to HBM (GB/s)", "value": value / 1e9, "unit": "GB/s", "n_gpus": 1,
        "steps": n, "warmup": 1, "ms_per_step": (load_s + reg_s) * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded normals, page-cached file)",
        "config": {"workload": f"one MoE layer of model.bin (gate + {E} experts x w1/w2/w3, fp32, "
                               f"{nbytes / 1e6:.0f} MB): index parse + every tensor to HBM, then bf16 registration",
                   "bytes": nbytes},
        "roofline": {"bound": "pcie", "achieved": value / 1e9, "peak": h2d / 1e9, "unit": "GB/s",
                     "frac": value / h2d, "traffic": None,
                     "note": "peak = this box's measured pinned host-to-device copy rate"},
        "cpu_baseline": None,
        "stages": {"load_ms": load_s * 1e3, "register_bf16_ms": reg_s * 1e3, "h2d_pinned_GB_s": h2d / 1e9},
    }), flush=True)


def cpp_c4_bench(args):
    """--config c4 --host cpp: the same prefill through the C++ drop-in
    (PhiTinyMoEModel::generate, as the reference harness calls it,
    src/main.cpp:585-594): a 32-layer model built from parts (random-init
    weights of the same distributions, fp32 tensors copied into the C++
    Tensors, bf16 experts registered by PhiMoE), each step one generate() on
    C4's 16 prompts (host trie and upload included)."""
    import torch
    from aps2026_amd import capi, synth

    if args.proj != "fp32":
        raise SystemExit("--host cpp runs the default build's fp32 projections")
    dev = torch.device("cuda:0")
    H, F, E, V, nl = 4096, 448, 16, 32064, 32
    drive_path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests", "cpp", "libmodel_drive.so")
    if not os.path.exists(drive_path):
        raise SystemExit(f"{drive_path} is not built (python -m aps2026_amd.build)")
    D = ctypes.CDLL(drive_path)
    D.md_model_create.restype = ctypes.c_void_p
    D.md_model_create.argtypes = [ctypes.c_int] * 8 + [ctypes.POINTER(ctypes.c_char_p),
                                                       ctypes.POINTER(ctypes.c_void_p), ctypes.c_int]
    D.md_generate.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int),
                              ctypes.c_int, ctypes.c_void_p, ctypes.POINTER(ctypes.c_double)]
    D.md_model_free.argtypes = [ctypes.c_void_p]
    D.md_last_error.restype = ctypes.c_char_p
    g = torch.Generator(device=dev).manual_seed(11)
    rn = lambda *shape, s=0.02: (s * torch.randn(shape, generator=g, device=dev)).contiguous()
    W = {"model.embed_tokens.weight": rn(V, H, s=1.0), "model.norm.weight": torch.ones(H, device=dev),
         "model.norm.bias": torch.zeros(H, device=dev), "lm_head.weight": rn(V, H), "lm_head.bias": rn(V)}
    model = None
    for i in range(nl):
        p = f"model.layers.{i}."
        for nm in ("input_layernorm", "post_attention_layernorm"):
            W[p + nm + ".weight"] = torch.ones(H, device=dev)
            W[p + nm + ".bias"] = torch.zeros(H, device=dev)
        for nm, (o, k) in (("q_proj", (2048, H)), ("k_proj", (512, H)), ("v_proj", (512, H)), ("o_proj", (H, 2048))):
            W[p + f"self_attn.{nm}.weight"] = rn(o, k)
            W[p + f"self_attn.{nm}.bias"] = rn(o)
        m = p + "block_sparse_moe."
        W[m + "gate.weight"] = rn(E, H)
        for e in range(E):
            for nm, shp in (("w1", (F, H)), ("w3", (F, H)), ("w2", (H, F))):
                W[m + f"experts.{e}.{nm}.weight"] = rn(*shp)
    names = list(W.keys())
    torch.cuda.synchronize()
    model = D.md_model_create(nl, H, V, E, F, 2048, 512, len(names),
                              (ctypes.c_char_p * len(names))(*[n.encode() for n in names]),
                              (ctypes.c_void_p * len(names))(*[W[n].data_ptr() for n in names]), capi.DTYPE_BF16)
    if not model:
        raise RuntimeError(D.md_last_error().decode())
    del W  # the C++ model holds its own copies
    torch.cuda.empty_cache()
    prompts = synth.c4_prompts()
    tokens = sum(len(q) for q in prompts)
    ids = (ctypes.c_int * tokens)(*[t for q in prompts for t in q])
    lens = (ctypes.c_int * len(prompts))(*[len(q) for q in prompts])
    logits = torch.empty((len(prompts), V), dtype=torch.float32, device=dev)
    secs = ctypes.c_double(0.0)

    def step(i):
        if D.md_generate(model, ids, lens, len(prompts), ctypes.c_void_p(logits.data_ptr()), ctypes.byref(secs)):
            raise RuntimeError(D.md_last_error().decode())
    t_settle = time.perf_counter()
    n_settle = 0
    while time.perf_counter() - t_settle < args.settle:
        step(n_settle)
        n_settle += 1
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    per = []
    for i in range(args.steps):
        step(i)
        per.append(secs.value)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    line = {
        "metric": "whole-model prefill tokens/s", "value": tokens * args.steps / elapsed, "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "settle_steps": n_settle,
        "ms_per_step": elapsed / args.steps * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32 attention, bf16 experts",
        "data": "synthetic (seeded torch normals, random-init weights)",
        "config": {"workload": ("c4 through the C++ drop-in: PhiTinyMoEModel::generate (host trie, embedding "
                                "gather, 32 x PhiDecoderLayer::forward_carry, final LayerNorm, last rows, LM head) "
                                f"on 16 prompts x 1024 ids, hidden {H}, {E} bf16 experts of {F}, vocab {V}; "
                                f"value counts the {tokens} prompt tokens"),
                   "host": "cpp", "tokens": tokens, "hidden": H, "experts": E, "ffn": F, "layers": nl},
        "roofline": None, "cpu_baseline": None,
        "stages": {"generate_ms_median": statistics.median(per) * 1e3, "generate_ms_min": min(per) * 1e3},
    }
    print(json.dumps(line), flush=True)
    D.md_model_free(model)


def decoder_bench(args):
    """--config c3: one whole decoder layer (input LayerNorm, fp32 q/k/v
    projections with bias, RoPE, GQA-4 tree attention, o projection, residual
    add + LayerNorm, bf16 MoE block) on the 4096 prefix-trie rows of 8
    prompts x 512 random ids; steps chain forward_carry through LAYERS
    random-init layers in turn (each step's input is the previous step's
    output and carried residual), as consecutive layers of a prefill.
    --config c4: the whole 32-layer model's prefill (PhiTinyMoEModel::generate)
    on C4's 16 prompts x 1024 ids: per step the host prefix trie and its
    upload, the embedding gather of the 10,240 node rows, 32 layers, the
    final add+LayerNorm, the last-row gather and the LM head (vocab 32064)."""
    import torch
    from aps2026_amd import capi, decoder, synth
    from aps2026_amd.moe import NORM_EPS

    dev = torch.device("cuda:0")
    H, F, E, V = 4096, 448, 16, 32064
    c4 = args.config == "c4"
    g = torch.Generator(device=dev).manual_seed(11)
    stream = torch.cuda.current_stream(dev)
    sptr = ctypes.c_void_p(stream.cuda_stream)
    L = capi.lib()
    if c4 and args.host == "cpp":
        return cpp_c4_bench(args)
    if c4:
        prompts = synth.c4_prompts()
        nl = 32
        lws = [decoder.random_layer(H, F, E, dev, g) for _ in range(nl)]
        emb = torch.randn((V, H), generator=g, device=dev)
        head_w = (0.02 * torch.randn((V, H), generator=g, device=dev)).contiguous()
        head_b = (0.02 * torch.randn(V, generator=g, device=dev)).contiguous()
        model = decoder.Model(emb, torch.ones(H, device=dev), torch.zeros(H, device=dev), head_w, head_b, lws,
                              tc={"fp32": "off", "tc": "tc", "tc_all": "all"}[args.proj])
        plan = decoder.RowPlan.from_prompts(prompts, dev)
        T, tokens = plan.rows, plan.prompt_tokens

        def step(i):
            p = decoder.RowPlan.from_prompts(prompts, dev)  # the host trie and its upload, as generate() does
            model.prefill(p)
        layer0, bufs = model.layers[0], model.buffers(T)
    else:
        rng = np.random.default_rng(7)
        prompts = [rng.integers(0, V, 512).tolist() for _ in range(8)]
        plan = decoder.RowPlan.from_prompts(prompts, dev)
        T = tokens = plan.rows
        lws = [decoder.random_layer(H, F, E, dev, g) for _ in range(LAYERS)]
        layers = [decoder.DecoderLayer(w, {"fp32": None, "tc": 3, "tc_all": 4}[args.proj]) for w in lws]
        bufs = decoder.Buffers.allocate(T, H, lws[0].moe, dev)
        bufs.x.copy_(torch.randn((T, H), generator=g, device=dev))
        bufs.carry.zero_()
        layer0 = layers[0]

        def step(i):
            layers[i % LAYERS].forward_carry(bufs, plan, True, sptr)
    torch.cuda.synchronize()

    t_settle = time.perf_counter()
    n_settle = 0
    while time.perf_counter() - t_settle < args.settle:
        step(n_settle)
        n_settle += 1
        torch.cuda.synchronize()
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed / args.steps * 1e3

    # ---- one layer's stages with HIP events on the launch stream ----------
    def p(t):
        return ctypes.c_void_p(t.data_ptr())
    w = layer0.w
    eps = ctypes.c_float(NORM_EPS)
    cos_d, sin_d = decoder._device_table(dev, plan.max_len, 128, decoder.ROPE_THETA)
    def proj(src, names):   # the layer's own projection path (fp32 chains or the split products)
        layer0._project(bufs, src, names, sptr)
        return 0
    calls = [
        ("input_layer_norm", lambda: L.aps_add_layer_norm(p(bufs.x), p(bufs.carry), p(w.in_w), p(w.in_b), T, H, eps,
                                                           p(bufs.normed), sptr)),
        ("qkv_proj", lambda: proj(bufs.normed, (("q_proj", bufs.q, 2048), ("k_proj", bufs.k, 512),
                                                ("v_proj", bufs.v, 512)))),
        ("rope", lambda: L.aps_rope_tree(p(bufs.q), p(bufs.k), p(plan.pos), T, 16, 4, 128, p(cos_d), p(sin_d),
                                         cos_d.shape[0], sptr)),
        ("attention_tree", lambda: L.aps_attention_tree(p(bufs.q), p(bufs.k), p(bufs.v), p(bufs.att), p(plan.pos),
                                                        p(plan.anc), plan.max_len, T, 16, 4, 128,
                                                        decoder.SLIDING_WINDOW, sptr)),
        ("o_proj", lambda: proj(bufs.att, (("o_proj", bufs.carry, H),))),
        ("add_layer_norm", lambda: L.aps_add_layer_norm(p(bufs.carry), p(bufs.x), p(w.post_w), p(w.post_b), T, H,
                                                         eps, p(bufs.post), sptr)),
        ("moe_block", lambda: L.aps_moe_forward(w.moe.handle, p(bufs.post), capi.DTYPE_F32, p(w.gate), T, p(bufs.x),
                                                capi.DTYPE_F32, p(bufs.ws), bufs.ws.numel(), sptr)),
    ]
    times = {nm: [] for nm, _ in calls}
    for i in range(12):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(calls) + 1)]
        ev[0].record(stream)
        for k, (nm, c) in enumerate(calls):
            rc = c()
            if rc:
                raise RuntimeError(f"{nm}: {capi.last_error()}")
            ev[k + 1].record(stream)
        torch.cuda.synchronize()
        if i >= 2:
            for k, (nm, _) in enumerate(calls):
                times[nm].append(ev[k].elapsed_time(ev[k + 1]) * 1e-3)
    mt = {nm: statistics.mean(v) for nm, v in times.items()}
    qkv_flops = 2.0 * T * H * (2048 + 512 + 512)
    o_flops = 2.0 * T * 2048 * H
    windows = plan.pos.cpu().numpy().astype(np.int64) + 1
    attn_flops = float(np.minimum(windows, decoder.SLIDING_WINDOW).sum()) * 16 * 128 * 4
    stages = {
        "input_layer_norm": {"us": mt["input_layer_norm"] * 1e6,
                             "GB_s": 4.0 * T * H * 4 / mt["input_layer_norm"] / 1e9},
        "qkv_proj": {"us": mt["qkv_proj"] * 1e6, "TFLOP_s": qkv_flops / mt["qkv_proj"] / 1e12},
        "rope": {"us": mt["rope"] * 1e6},
        "attention_tree": {"us": mt["attention_tree"] * 1e6, "TFLOP_s": attn_flops / mt["attention_tree"] / 1e12},
        "o_proj": {"us": mt["o_proj"] * 1e6, "TFLOP_s": o_flops / mt["o_proj"] / 1e12},
        "add_layer_norm": {"us": mt["add_layer_norm"] * 1e6, "GB_s": 4.0 * T * H * 4 / mt["add_layer_norm"] / 1e9},
        "moe_block": {"us": mt["moe_block"] * 1e6},
        "layer_total_us": sum(mt.values()) * 1e6,
    }
    if c4:
        t_plan = []
        for _ in range(5):
            t1 = time.perf_counter()
            decoder.RowPlan.from_prompts(prompts, dev)
            torch.cuda.synchronize()
            t_plan.append(time.perf_counter() - t1)
        stages["prefix_trie_and_upload_ms"] = statistics.median(t_plan) * 1e3
    # the projections dominate: one fp32 FMA chain per output (the reference's
    # order) as chains of K = 1 fp32 MFMAs; MI355X's published fp32 matrix
    # rate is 157.3 TFLOP/s
    proj_s = mt["qkv_proj"] + mt["o_proj"]
    if layer0.tc:
        # the split products on the bf16 matrix cores: terms x the fp32
        # FLOPs of bf16 MFMA work per projection (the x split included in
        # the time), against the 2.5 PFLOP/s dense bf16 peak
        mma = layer0.tc_terms * (qkv_flops + o_flops)
        roofline = {"bound": "mfma", "kernel": f"k_linear_tc ({layer0.tc_terms} bf16 products, q/k/v/o projections)",
                    "achieved": mma / proj_s / 1e12, "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
                    "frac": mma / proj_s / PEAK_BF16, "traffic": None, "flops_per_launch": mma / 4,
                    "launch_us": proj_s / 4 * 1e6, "fp32_equivalent_TFLOP_s": (qkv_flops + o_flops) / proj_s / 1e12}
    else:
        roofline = {"bound": "mfma", "kernel": "k_linear_mfma (q/k/v/o projections)",
                    "achieved": (qkv_flops + o_flops) / proj_s / 1e12, "peak": PEAK_F32 / 1e12, "unit": "TFLOP/s",
                    "frac": (qkv_flops + o_flops) / proj_s / PEAK_F32, "traffic": None,
                    "flops_per_launch": (qkv_flops + o_flops) / 4, "launch_us": proj_s / 4 * 1e6}
    proj_text = {"fp32": "fp32 q/k/v/o projections with bias",
                 "tc": "split-bf16 q/k/v/o projections (three bf16 products, the reference's USE_TC arithmetic"
                       + (", on the LM head and layer 31 as USE_TC selects" if c4 else "") + ")",
                 "tc_all": "split-bf16 q/k/v/o projections on every layer and the LM head (four bf16 products, "
                           "USE_TC_ALL)"}[args.proj]
    workload = (f"c4: whole 32-layer random-init model prefill (generate): 16 prompts x 1024 ids, groups of 4 "
                f"sharing a 512-id prefix, host prefix trie + upload, embedding gather of {T} node rows, 32 "
                f"decoder layers (LayerNorm+bias, {proj_text}, 16/4 heads of 128, RoPE, "
                f"GQA tree attention, bf16 MoE: hidden {H}, {E} experts top-2, ffn {F}), final add+LayerNorm, "
                f"last-row gather, LM head (vocab {V}); value counts the {tokens} prompt tokens"
                if c4 else
                f"c3: one whole decoder layer on the {T} prefix-trie rows of 8 prompts x 512 random ids "
                f"(LayerNorm+bias, {proj_text}, 16/4 heads of 128, RoPE, GQA tree "
                f"attention, residual add+LayerNorm, bf16 MoE: hidden {H}, {E} experts top-2, ffn {F}); steps "
                f"chain forward_carry through {LAYERS} random-init layers")
    line = {
        "metric": "whole-model prefill tokens/s" if c4 else "decoder-layer prefill tokens/s",
        "value": tokens * args.steps / elapsed, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "settle_steps": n_settle, "ms_per_step": ms_per_step, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 attention, bf16 experts" + ("" if args.proj == "fp32" else
                                                  f", split-bf16 projections ({'four' if args.proj == 'tc_all' else 'three'} products)"),
        "data": "synthetic (seeded torch normals, random-init weights)",
        "config": {"workload": workload, "tokens": tokens, "rows": T, "hidden": H, "experts": E, "ffn": F,
                   "layers": 32 if c4 else LAYERS},
        "roofline": roofline, "cpu_baseline": None, "stages": stages,
    }
    print(json.dumps(line), flush=True)
    for lw in lws:
        lw.release()


PROBE_LIB = os.path.join(ROOT, "aps2026_amd", "probe", "libaps_probe.so")


def fma_chain_costs():
    """fp32 FMA chain costs on this device, from aps_probe_fma_chain
    (aps2026_amd/probe/fma_chain.hip; one workgroup per CU, 8192 steps):
    dependent v_fmac_f32 at one wave per SIMD (the chain latency),
    dependent v_fmac_f32_dpp (the router's instruction), and independent
    FMAs at four waves per SIMD (the SIMD's issue interval per wave
    instruction: cycles per wave / 4); shader clock in MHz."""
    if not os.path.exists(PROBE_LIB):
        raise RuntimeError(f"{PROBE_LIB} is not built (python -m aps2026_amd.build)")
    L = ctypes.CDLL(PROBE_LIB)
    L.aps_probe_fma_chain.argtypes = [ctypes.c_int] * 4 + [ctypes.POINTER(ctypes.c_double)] * 2

    def run(waves_per_simd, dpp, chains):
        cyc, mhz = ctypes.c_double(0.0), ctypes.c_double(0.0)
        rc = L.aps_probe_fma_chain(waves_per_simd, dpp, chains, 8192, ctypes.byref(cyc), ctypes.byref(mhz))
        if rc != 0:
            raise RuntimeError(f"aps_probe_fma_chain: HIP error {rc}")
        return cyc.value, mhz.value

    dep, mhz = run(1, 0, 1)
    dep_dpp, _ = run(1, 1, 1)
    ind4, _ = run(4, 0, 2)
    return {"dependent_cycles": dep, "dependent_dpp_cycles": dep_dpp, "simd_issue_cycles": ind4 / 4.0,
            "clock_mhz": mhz}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (--gpus {args.gpus} requested); "
              "multi-GPU sharding is designed but not built", file=sys.stderr)
        sys.exit(2)
    if args.config == "load":
        load_bench(args)
        return
    if args.config in ("c3", "c4"):
        decoder_bench(args)
        return

    import torch
    from aps2026_amd import capi, moe, synth

    dev = torch.device("cuda:0")
    inp = synth.make_config(args.config)
    T, H, E, F = inp.T, inp.H, inp.E, inp.F
    A = 2 * T
    fp8 = inp.dtype == "fp8"
    bf16 = inp.dtype in ("bf16", "fp8")        # x and outputs are bf16 on both MFMA paths
    tdt = torch.bfloat16 if bf16 else torch.float32

    def dev_bits(bits):
        return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(torch.bfloat16)

    if bf16:
        x = dev_bits(inp.packed["x_bf16"])
    else:
        x = torch.from_numpy(inp.x).to(dev)
    gate = torch.from_numpy(inp.gate).to(dev)
    layers = []
    for _ in range(LAYERS):
        lists, scales = [], []
        for nm in ("w1", "w2", "w3"):
            if fp8:
                d = torch.from_numpy(inp.packed[nm + "_e4m3"]).to(dev)
                sc = torch.from_numpy(inp.packed[nm + "_scale"]).to(dev)
                scales.append([sc[e].contiguous() for e in range(E)])
            elif bf16:
                d = dev_bits(inp.packed[nm + "_bf16"])
            else:
                d = torch.from_numpy(getattr(inp, nm)).to(dev)
            lists.append([d[e].contiguous() for e in range(E)])
        if fp8:
            layers.append(moe.register_moe_weights_gpu(*lists, compute_dtype=moe.FP8, scales=tuple(scales)))
        else:
            layers.append(moe.register_moe_weights_gpu(*lists, compute_dtype=tdt))
        del lists, scales
    torch.cuda.synchronize()

    if args.copy_probe:
        src = torch.full((COPY_PROBE_BYTES,), 7, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    L = capi.lib()
    lay = layers[0].layout(T)
    ws = torch.empty(lay.total_bytes, dtype=torch.uint8, device=dev)
    out = torch.empty((T, H), dtype=tdt, device=dev)
    stream = torch.cuda.current_stream(dev)
    sptr = ctypes.c_void_p(stream.cuda_stream)
    xd = capi.DTYPE_BF16 if bf16 else capi.DTYPE_F32
    args_fwd = [(w.handle, ctypes.c_void_p(x.data_ptr()), xd, ctypes.c_void_p(gate.data_ptr()), T,
                 ctypes.c_void_p(out.data_ptr()), xd, ctypes.c_void_p(ws.data_ptr()), ws.numel(), sptr)
                for w in layers]
    def step(i):
        rc = L.aps_moe_forward(*args_fwd[i % LAYERS])
        if rc:
            raise RuntimeError(capi.last_error())

    t_settle = time.perf_counter()
    n_settle = 0
    while time.perf_counter() - t_settle < args.settle:
        for _ in range(LAYERS):
            step(n_settle)
            n_settle += 1
        torch.cuda.synchronize()
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed / args.steps * 1e3
    tokens_per_s = T * args.steps / elapsed

    # ---- per-stage timing with HIP events on the launch stream ------------
    def p(t):
        return ctypes.c_void_p(t.data_ptr())

    logits = torch.empty((T, E), dtype=torch.float32, device=dev)
    routes = torch.empty((T, 2), dtype=torch.uint8, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    arows = torch.empty(A, dtype=torch.int32, device=dev)
    rpos = torch.empty(A, dtype=torch.int32, device=dev)
    scratch = torch.empty(max(L.aps_moe_dispatch_workspace_size(T, E), 1), dtype=torch.uint8, device=dev)
    act = torch.empty((A, F), dtype=tdt, device=dev)
    y = torch.empty((A, H), dtype=tdt, device=dev)
    if fp8:
        kp = (F + 127) // 128 * 128
        xq = torch.empty((T, H), dtype=torch.uint8, device=dev)
        xs = torch.empty(T, dtype=torch.float32, device=dev)
        actq = torch.empty((A, kp), dtype=torch.uint8, device=dev)
        acts = torch.empty(A, dtype=torch.float32, device=dev)
        stages = ["router_logits", "route_top2", "dispatch", "quant_x", "ffn_up", "quant_act", "ffn_down",
                  "combine"]
    else:
        stages = ["router_logits", "route_top2", "dispatch", "ffn_up", "ffn_down", "combine"]
    times = {s: [] for s in stages}
    n_stage = max(args.steps, 10)
    for i in range(n_stage + 2):
        w = layers[i % LAYERS]
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)]
        ev[0].record(stream)
        calls = [
            lambda: L.aps_router_logits(p(x), xd, p(gate), T, H, E, p(logits), sptr),
            lambda: L.aps_moe_route_top2(p(logits), T, E, p(routes), sptr),
            lambda: L.aps_moe_dispatch(p(routes), T, E, p(counts), p(offsets), p(arows), p(rpos), p(scratch),
                                       scratch.numel(), sptr),
        ]
        if fp8:
            calls += [
                lambda: L.aps_quantise_rows_e4m3(p(x), H, H, p(xq), H, p(xs), T, sptr),
                lambda: L.aps_moe_ffn_up_fp8(w.handle, p(xq), p(xs), T, p(offsets), p(arows), p(act), sptr),
                lambda: L.aps_quantise_rows_e4m3(p(act), F, F, p(actq), kp, p(acts), A, sptr),
                lambda: L.aps_moe_ffn_down_fp8(w.handle, p(actq), p(acts), T, p(offsets), p(y), sptr),
            ]
        else:
            calls += [
                lambda: L.aps_moe_ffn_up(w.handle, p(x), xd, T, p(offsets), p(arows), p(act), None, sptr),
                lambda: L.aps_moe_ffn_down(w.handle, p(act), None, T, p(offsets), p(y), sptr),
            ]
        calls.append(lambda: L.aps_moe_combine(p(y), xd, p(rpos), T, H, p(out), xd, sptr))
        for k, c in enumerate(calls):
            rc = c()
            if rc:
                raise RuntimeError(f"{stages[k]}: {capi.last_error()}")
            ev[k + 1].record(stream)
        torch.cuda.synchronize()
        if i >= 2:
            for k, s in enumerate(stages):
                times[s].append(ev[k].elapsed_time(ev[k + 1]) * 1e-3)
    mean_t = {s: statistics.mean(v) for s, v in times.items()}

    esz = 2 if bf16 else 4
    flops_up = 4.0 * A * H * F
    flops_down = 2.0 * A * F * H
    peak = PEAK_FP8 if fp8 else (PEAK_BF16 if bf16 else PEAK_F32)
    bytes_router = T * H * esz + E * H * 4 + T * E * 4
    bytes_combine = A * H * esz + T * H * esz + A * 4
    # The router's bound is its FMA chains, not HBM: every logit is one fp32
    # FMA chain over H steps in the reference's order, one chain per lane.
    # Floor per step: the dependent-FMA latency of one wave, or, when the
    # T*E chains need several waves per SIMD, that many wave instructions at
    # the SIMD's issue interval; both measured on this device at its
    # sustained clock (aps2026_amd/probe/fma_chain.hip).
    n_cu = torch.cuda.get_device_properties(dev).multi_processor_count
    fma = fma_chain_costs()
    waves_per_simd = -(-T * E // (n_cu * 4 * 64))
    floor_cycles = max(fma["dependent_cycles"], waves_per_simd * fma["simd_issue_cycles"])
    chain_floor_s = H * floor_cycles / (fma["clock_mhz"] * 1e6)
    stage_report = {
        "router_logits": {"us": mean_t["router_logits"] * 1e6,
                          "GB_s": bytes_router / mean_t["router_logits"] / 1e9,
                          "chain_floor_us": chain_floor_s * 1e6,
                          "frac_of_chain_floor": chain_floor_s / mean_t["router_logits"],
                          "cycles_per_step": mean_t["router_logits"] * fma["clock_mhz"] * 1e6 / H,
                          "fma_chain_probe": {**fma, "waves_per_simd": waves_per_simd}},
        "route_top2": {"us": mean_t["route_top2"] * 1e6},
        "dispatch": {"us": mean_t["dispatch"] * 1e6},
        "ffn_up": {"us": mean_t["ffn_up"] * 1e6, "TFLOP_s": flops_up / mean_t["ffn_up"] / 1e12},
        "ffn_down": {"us": mean_t["ffn_down"] * 1e6, "TFLOP_s": flops_down / mean_t["ffn_down"] / 1e12},
        "combine": {"us": mean_t["combine"] * 1e6, "GB_s": bytes_combine / mean_t["combine"] / 1e9},
        **({"quant_x": {"us": mean_t["quant_x"] * 1e6}, "quant_act": {"us": mean_t["quant_act"] * 1e6}}
           if fp8 else {}),
        "grouped_gemm_total_TFLOP_s": (flops_up + flops_down) / (mean_t["ffn_up"] + mean_t["ffn_down"]) / 1e12,
    }
    achieved = flops_up / mean_t["ffn_up"]
    kname = "k_ffn_up<Fp8Fmt>" if fp8 else ("k_ffn_up<Bf16Fmt>" if bf16 else "k_ffn_up_f32")
    roofline = {"bound": "mfma", "kernel": kname,
                "achieved": achieved / 1e12, "peak": peak / 1e12, "unit": "TFLOP/s",
                "frac": achieved / peak,
                "traffic": (TRAFFIC_KIB[args.config][0] * FETCH_SCALE + TRAFFIC_KIB[args.config][1] * WRITE_SCALE) * 1024
                if args.config in TRAFFIC_KIB else None,
                "flops_per_launch": flops_up, "launch_us": mean_t["ffn_up"] * 1e6}

    # ---- CPU baseline: the reference CPU-path algorithm on the host cores ----
    cpu = None
    if args.cpu_baseline == "auto":
        import oracle
        runs = []
        oracle.moe_forward(inp.x[:256], inp.gate, inp.w1, inp.w3, inp.w2)  # warm-up
        while len(runs) < 2 or sum(runs) < args.cpu_seconds:
            t = time.perf_counter()
            oracle.moe_forward(inp.x, inp.gate, inp.w1, inp.w3, inp.w2)
            runs.append(time.perf_counter() - t)
        total = sum(runs)
        cpu = {"value": T * len(runs) / total, "unit": "tokens/s", "cores": oracle.num_threads(), "kind": "port",
               "host_cpus_visible": len(os.sched_getaffinity(0)),
               "sample": f"{len(runs)} runs of the full {args.config} batch ({T} tokens each, {total:.1f} s in "
                         f"all, median {statistics.median(runs):.2f} s), values upcast to fp32, reference "
                         f"CPU-path order (router, route, per-expert gather/FFN/scatter-add), after a 256-token "
                         f"warm-up; cores = OpenMP threads used (omp_get_max_threads); the timed code is the "
                         f"oracle's blocked, transposed restatement, faster than the reference's plain "
                         f"omp-parallel loops"}

    line = {
        "metric": METRIC, "value": tokens_per_s, "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "settle_steps": n_settle, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8" if fp8 else ("bf16" if bf16 else "f32"), "data": "synthetic (seeded PCG64 normals, random-init weights)",
        "config": {"workload": (f"{args.config}: MoE FFN block, {T} tokens, hidden {H}, {E} experts top-2, "
                                f"ffn {F}, {inp.dtype}" + (", Zipf(1.1) expert loads" if inp.zipf else "")),
                   "tokens": T, "rows": T, "hidden": H, "experts": E, "ffn": F, "layers_rotated": LAYERS},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "stages": stage_report,
    }
    print(json.dumps(line), flush=True)
    for w in layers:
        w.release()


if __name__ == "__main__":
    main()
