"""GPU parity of the HIP MoE path against the CPU oracle, through the C ABI.

Bars (the tolerances stated for this path):
  routing indices, per-expert counts, offsets and permutation: bit-exact
  fp32 path (config C1): output within 1e-5 relative, normwise per row
  bf16 path (config C2): output within 2e-2 relative, normwise per row
At C2's full size the oracle checks routing bit for bit on every token, every
one of the 2T expert outputs and every block output row; determinism across
runs and the staged and fused entry points agreeing bit for bit are checked
besides.
"""
import sys

import numpy as np
import pytest
import torch

import oracle
from aps2026_amd import capi, moe, synth

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5
TOL_BF16 = 2e-2


def note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def to_dev_bf16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(torch.bfloat16)


def bf16_to_np(t):
    return synth.bf16_bits_to_f32(t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16))


def as_np_f32(t):
    return bf16_to_np(t) if t.dtype == torch.bfloat16 else t.float().cpu().numpy()


def weights_for(inp, dev, compute=None, src=None):
    compute = compute or (torch.float32 if inp.dtype == "f32" else torch.bfloat16)
    src = src or ("bf16" if inp.dtype == "bf16" else "f32")
    lists = []
    for nm in ("w1", "w2", "w3"):
        if src == "bf16":
            b = to_dev_bf16(inp.packed[nm + "_bf16"], dev)
        else:
            b = torch.from_numpy(getattr(inp, nm)).to(dev)
        lists.append([b[e].contiguous() for e in range(inp.E)])
    return moe.register_moe_weights_gpu(lists[0], lists[1], lists[2], compute_dtype=compute)


def x_for(inp, dev):
    if inp.dtype == "f32":
        return torch.from_numpy(inp.x).to(dev)
    return to_dev_bf16(inp.packed["x_bf16"], dev)


def rowwise_err(got, ref):
    num = np.linalg.norm(got.astype(np.float64) - ref.astype(np.float64), axis=1)
    den = np.maximum(np.linalg.norm(ref.astype(np.float64), axis=1), 1e-30)
    return num / den


def check_plan(plan, ref, T):
    np.testing.assert_array_equal(plan["routes"].cpu().numpy().astype(np.int32), ref["routes"])
    np.testing.assert_array_equal(plan["counts"].cpu().numpy().view(np.uint32), ref["counts"])
    np.testing.assert_array_equal(plan["offsets"].cpu().numpy().view(np.uint32), ref["offsets"])
    np.testing.assert_array_equal(plan["assignment_rows"].cpu().numpy().view(np.uint32), ref["assignment_rows"])
    np.testing.assert_array_equal(plan["route_positions"].cpu().numpy().view(np.uint32), ref["route_positions"])


def oracle_routing(inp):
    logits = oracle.router_logits(inp.x, inp.gate)
    routes = oracle.route_top2(logits)
    counts, offsets, rows, pos = oracle.dispatch(routes, inp.E)
    return dict(logits=logits, routes=routes, counts=counts, offsets=offsets,
                assignment_rows=rows, route_positions=pos)


def full_oracle_ffn(inp, ref):
    """Oracle expert outputs for all 2T positions (position order: token
    assignment_rows[p] through expert e for p in [offsets[e], offsets[e+1]))
    and the oracle combine of them for all T tokens."""
    rows = ref["assignment_rows"].astype(np.int64)
    experts = np.repeat(np.arange(inp.E, dtype=np.int32), ref["counts"].astype(np.int64))
    y_ref = oracle.ffn_rows(inp.x[rows], experts, inp.w1, inp.w3, inp.w2)
    out_ref = oracle.combine(y_ref, ref["routes"], ref["route_positions"])
    return y_ref, out_ref


# ---------------------------------------------------------------------------

def test_c1_fp32_full_parity(gpu_device):
    note("C1 fp32 T=512 full block vs oracle")
    inp = synth.make_config("c1")
    w = weights_for(inp, gpu_device)
    x, gate = x_for(inp, gpu_device), torch.from_numpy(inp.gate).to(gpu_device)
    out = moe.moe_forward_gpu(x, gate, w, out_dtype=torch.float32)
    plan = w.plan_views(inp.T)
    torch.cuda.synchronize()
    ref = oracle.reference_path(inp.x, inp.gate, inp.w1, inp.w3, inp.w2)
    np.testing.assert_array_equal(plan["logits"].cpu().numpy().view(np.uint32), ref["logits"].view(np.uint32))
    check_plan(plan, ref, inp.T)
    y = plan["y"].cpu().numpy()
    assert rowwise_err(y, ref["y"]).max() <= TOL_F32
    got = out.cpu().numpy()
    err = rowwise_err(got, ref["out"])
    same = np.mean(got.view(np.uint32) == ref["out"].view(np.uint32))
    note(f"C1 max normwise err {err.max():.3e}, bit-identical fraction {same:.6f}")
    assert err.max() <= TOL_F32
    w.release()


def test_c2_bf16_zipf_parity(gpu_device):
    note("C2 bf16 T=4096 Zipf(1.1): routing, every expert output and every block output row")
    inp = synth.make_config("c2")
    w = weights_for(inp, gpu_device)
    x, gate = x_for(inp, gpu_device), torch.from_numpy(inp.gate).to(gpu_device)
    out = moe.moe_forward_gpu(x, gate, w, out_dtype=torch.bfloat16)
    plan = w.plan_views(inp.T)
    torch.cuda.synchronize()
    ref = oracle_routing(inp)
    np.testing.assert_array_equal(plan["logits"].cpu().numpy().view(np.uint32), ref["logits"].view(np.uint32))
    check_plan(plan, ref, inp.T)
    counts = ref["counts"].astype(np.int64)
    note(f"C2 counts {counts.tolist()} top/mean {counts.max() / counts.mean():.2f}")

    # every one of the 2T expert outputs, in position order, and every one of
    # the T block output rows against the oracle's FFN and combine
    y_ref, out_ref = full_oracle_ffn(inp, ref)
    y_gpu = bf16_to_np(plan["y"])
    e_y = rowwise_err(y_gpu, y_ref)
    got = bf16_to_np(out)
    e_o = rowwise_err(got, out_ref)
    note(f"C2 all {2 * inp.T} positions max normwise err {e_y.max():.3e}; "
         f"all {inp.T} output rows max {e_o.max():.3e}")
    assert e_y.max() <= TOL_BF16
    assert e_o.max() <= TOL_BF16
    assert np.isfinite(got).all()
    w.release()


def test_large_batch_65536_tokens(gpu_device):
    """A batch 16x C2 (65,536 tokens, bf16, Zipf loads): 8,192-row expert
    groups, work lists of thousands of tiles, a 1024-tile histogram.  Logits
    and the whole routing plan bit-exact; expert FFN and block output on a
    sample of tokens within the bf16 bar."""
    T = 65536
    note(f"large batch T={T}")
    inp = synth.make_config("c2", T=T)
    w = weights_for(inp, gpu_device)
    x, gate = x_for(inp, gpu_device), torch.from_numpy(inp.gate).to(gpu_device)
    out = moe.moe_forward_gpu(x, gate, w, out_dtype=torch.bfloat16)
    plan = w.plan_views(T)
    torch.cuda.synchronize()
    ref = oracle_routing(inp)
    np.testing.assert_array_equal(plan["logits"].cpu().numpy().view(np.uint32), ref["logits"].view(np.uint32))
    check_plan(plan, ref, T)
    rng = np.random.default_rng(1)
    toks = np.unique(np.concatenate([np.arange(16), np.arange(T - 16, T), rng.choice(T, 96, replace=False)]))
    y_ref = oracle.ffn_rows(np.repeat(inp.x[toks], 2, axis=0), ref["routes"][toks].reshape(-1), inp.w1, inp.w3,
                            inp.w2)
    out_ref = (0.5 * (y_ref[0::2].astype(np.float64) + y_ref[1::2])).astype(np.float32)
    err = rowwise_err(bf16_to_np(out)[toks], out_ref)
    note(f"large batch sample max normwise err {err.max():.3e}")
    assert err.max() <= TOL_BF16
    w.release()


@pytest.mark.parametrize("y_dtype,out_dtype", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                               (torch.float32, torch.float32), (torch.float32, torch.bfloat16)])
def test_combine_signed_zeros_and_special_values(gpu_device, y_dtype, out_dtype):
    """aps_moe_combine against the oracle's literal (0 + 0.5 a) + 0.5 b
    (k_moe_combine): token pairs of -0/-0 (the reference gives +0), -0/+0,
    -0/x, subnormals, the largest finite values (0.5 a + 0.5 b stays finite),
    infinities and NaN, beside random values; bit for bit, NaN as NaN."""
    rng = np.random.default_rng(21)
    T, H = 300, 256
    y = rng.standard_normal((2 * T, H)).astype(np.float32)
    special = np.array([-0.0, 0.0, -0.0, 1.5, 1e-40, -1e-40, 3.3e38, 3.3e38, np.inf, -np.inf, np.nan, 2.0],
                       np.float32)
    pos = rng.permutation(2 * T).astype(np.uint32)
    for k in range(len(special)):
        for j in range(len(special)):
            t = (k * len(special) + j) % T
            y[pos[2 * t], k * 16 + j] = special[k]
            y[pos[2 * t + 1], k * 16 + j] = special[j]
    if y_dtype == torch.bfloat16:
        y = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(y))   # the values a bf16 y holds
        y_dev = torch.from_numpy(synth.f32_to_bf16_bits(y).view(np.int16)).to(gpu_device).view(torch.bfloat16)
    else:
        y_dev = torch.from_numpy(y).to(gpu_device)
    routes = np.zeros((T, 2), np.int32)
    routes[:, 1] = 1
    want = oracle.combine(y, routes, pos)
    got = moe.combine(y_dev, torch.from_numpy(pos.view(np.int32)).to(gpu_device), T, out_dtype=out_dtype)
    torch.cuda.synchronize()
    if out_dtype == torch.bfloat16:
        got = synth.bf16_bits_to_f32(got.view(torch.int16).cpu().numpy().view(np.uint16))
        want = synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(want))
    else:
        got = got.cpu().numpy()
    nan = np.isnan(want)
    np.testing.assert_array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got.view(np.uint32)[~nan], want.view(np.uint32)[~nan])
    # the -0/-0 pairs (special values 0 and 2) gave +0
    for k, j in ((0, 0), (0, 2), (2, 0), (2, 2)):
        t = (k * len(special) + j) % T
        assert got.view(np.uint32)[t, k * 16 + j] == 0, (k, j)


def test_c2_deterministic_and_entry_points_agree(gpu_device):
    note("C2 determinism + fused vs grouped vs staged entry points (T=1024)")
    inp = synth.make_config("c2", T=1024)
    w = weights_for(inp, gpu_device)
    x, gate = x_for(inp, gpu_device), torch.from_numpy(inp.gate).to(gpu_device)
    a = moe.moe_forward_gpu(x, gate, w).clone()
    b = moe.moe_forward_gpu(x, gate, w).clone()
    logits = torch.empty((inp.T, inp.E), dtype=torch.float32, device=gpu_device)
    moe.matmul_transposed_gpu(x, gate, logits)
    c = moe.moe_forward_grouped_gpu(x, logits, w).clone()
    routes = moe.route_top2(logits)
    counts, offsets, arows, rpos = moe.dispatch(routes, inp.E)
    y = moe.expert_ffn(w, x, offsets, arows)
    d = moe.combine(y, rpos, inp.T, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    for other in (b, c, d):
        assert torch.equal(a.view(torch.int16), other.view(torch.int16))
    w.release()


@pytest.mark.parametrize("E", [2, 8, 16, 24, 32, 48, 64])
@pytest.mark.parametrize("H", [256, 1280, 2048])
def test_router_kernel_shapes(gpu_device, E, H):
    """Every router kernel variant: 1, 2 or 4 rows of 16 lanes per token
    (E <= 16 / 32 / 64), ring stages of 4, 2 or 1 windows of 128 steps, an
    odd stage count (H = 1280), fp32 and bf16 x.  Logits bit-exact from the
    staged entry point; logits, routes, counts and permutation bit-exact from
    the fused forward, whose router also writes the routes and the tile
    histogram.  T = 333 leaves a partial 16-token workgroup and a partial
    64-token tile."""
    T = 333
    for dtype in ("f32", "bf16"):
        note(f"router T={T} H={H} E={E} x {dtype}")
        inp = synth.make_moe_inputs(T=T, H=H, E=E, F=64, dtype=dtype, seed=7 * E + H)
        x, gate = x_for(inp, gpu_device), torch.from_numpy(inp.gate).to(gpu_device)
        ref = oracle_routing(inp)
        logits = torch.full((T, E), float("nan"), dtype=torch.float32, device=gpu_device)
        moe.matmul_transposed_gpu(x, gate, logits)
        w = weights_for(inp, gpu_device)
        moe.moe_forward_gpu(x, gate, w)
        plan = w.plan_views(T)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(logits.cpu().numpy().view(np.uint32), ref["logits"].view(np.uint32))
        np.testing.assert_array_equal(plan["logits"].cpu().numpy().view(np.uint32), ref["logits"].view(np.uint32))
        check_plan(plan, ref, T)
        w.release()


@pytest.mark.parametrize("E,T", [(16, 8192), (16, 5000), (8, 4097), (2, 7777), (16, 10240), (12, 12345)])
def test_router_32_token_workgroups(gpu_device, E, T):
    """Batches of 4,097 .. 8,192 tokens with E <= 16 (on a 256-CU MI355X)
    take the eight-wave router, 32 tokens per workgroup, two quarter-tile
    bytes of the histogram each (7,777 leaves a partial workgroup and a
    partial tile); the larger batches (10,240 and 12,345 tokens) go back to
    16-token workgroups.  Logits bit-exact from the staged entry point; logits,
    routes, counts and permutation bit-exact from the fused forward; fp32 x
    with bf16 experts (the router also writes the FFN's bf16 copy of x)
    gives the same output as the grouped entry point, which converts x on
    its own."""
    H = 1024
    for dtype, compute in (("bf16", None), ("f32", torch.float32), ("f32", torch.bfloat16)):
        note(f"router 32-token workgroups T={T} E={E} x {dtype} experts {compute}")
        inp = synth.make_moe_inputs(T=T, H=H, E=E, F=64, dtype=dtype, seed=11 * E + T)
        x, gate = x_for(inp, gpu_device), torch.from_numpy(inp.gate).to(gpu_device)
        ref = oracle_routing(inp)
        logits = torch.full((T, E), float("nan"), dtype=torch.float32, device=gpu_device)
        moe.matmul_transposed_gpu(x, gate, logits)
        w = weights_for(inp, gpu_device, compute=compute)
        fused = moe.moe_forward_gpu(x, gate, w).clone()
        plan = w.plan_views(T)
        grouped = moe.moe_forward_grouped_gpu(x, logits, w)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(logits.cpu().numpy().view(np.uint32), ref["logits"].view(np.uint32))
        np.testing.assert_array_equal(plan["logits"].cpu().numpy().view(np.uint32), ref["logits"].view(np.uint32))
        check_plan(plan, ref, T)
        assert torch.equal(fused.view(torch.int32 if fused.dtype == torch.float32 else torch.int16),
                           grouped.view(torch.int32 if grouped.dtype == torch.float32 else torch.int16))
        w.release()


@pytest.mark.parametrize("E,T", [(16, 20000), (24, 5000), (64, 9000), (2, 3000), (16, 1 << 20)])
def test_dispatch_many_tiles(gpu_device, E, T):
    """The staged dispatch on random routes over many 64-token tiles (more
    than one batch of histogram loads per wave, partial last workgroup),
    bit-exact against the oracle's stable counting sort."""
    note(f"dispatch E={E} T={T}")
    rng = np.random.default_rng(E * 1000 + T)
    first = rng.integers(0, E, T)
    second = (first + rng.integers(1, E, T)) % E
    routes = np.stack([first, second], axis=1).astype(np.uint8)
    want = oracle.dispatch(routes, E)
    got = moe.dispatch(torch.from_numpy(routes).to(gpu_device), E)
    torch.cuda.synchronize()
    for g, w_ in zip(got, want):
        np.testing.assert_array_equal(g.cpu().numpy().astype(np.uint32), w_)


@pytest.mark.parametrize("E,T", [(16, 5000), (2, 700)])
def test_dispatch_caller_routes_out_of_contract(gpu_device, E, T):
    """Caller routes the router never writes: a token whose two slots name
    one expert takes two consecutive positions of it (slot 0 first), which
    is the oracle's stable sort of the (token, slot) pairs; ids >= E are
    treated as E - 1 and counted.  Every index stays in range."""
    note(f"dispatch out-of-contract routes E={E} T={T}")
    rng = np.random.default_rng(E + T)
    routes = rng.integers(0, E, (T, 2))
    routes[::7, 1] = routes[::7, 0]                    # repeated expert
    big = rng.choice(T, 40, replace=False)
    routes[big, rng.integers(0, 2, 40)] = rng.integers(E, 256, 40)  # ids >= E
    n_big = int((routes >= E).sum())
    clamped = np.minimum(routes, E - 1)
    want = oracle.dispatch(clamped.astype(np.uint8), E)
    dev_routes = torch.from_numpy(routes.astype(np.uint8)).to(gpu_device)
    with pytest.raises(ValueError, match=f"{n_big} route ids"):
        moe.dispatch(dev_routes, E)
    got = moe.dispatch(dev_routes, E, check_ids=False)
    torch.cuda.synchronize()
    for g, w_ in zip(got, want):
        np.testing.assert_array_equal(g.cpu().numpy().astype(np.uint32), w_)
    # valid routes leave the counter at zero
    ok = moe.dispatch(torch.from_numpy(clamped.astype(np.uint8)).to(gpu_device), E)
    for g, w_ in zip(ok, want):
        np.testing.assert_array_equal(g.cpu().numpy().astype(np.uint32), w_)


@pytest.mark.parametrize("T", [1, 2, 3, 63, 64, 65, 127, 129, 300])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_ragged_rows_small_shapes(gpu_device, T, dtype):
    note(f"ragged T={T} {dtype} H=256 F=64 E=16")
    inp = synth.make_moe_inputs(T=T, H=256, E=16, F=64, dtype=dtype, seed=100 + T)
    w = weights_for(inp, gpu_device)
    x, gate = x_for(inp, gpu_device), torch.from_numpy(inp.gate).to(gpu_device)
    out = moe.moe_forward_gpu(x, gate, w, out_dtype=torch.float32)
    plan = w.plan_views(T)
    torch.cuda.synchronize()
    ref = oracle.reference_path(inp.x, inp.gate, inp.w1, inp.w3, inp.w2)
    np.testing.assert_array_equal(plan["logits"].cpu().numpy().view(np.uint32), ref["logits"].view(np.uint32))
    check_plan(plan, ref, T)
    tol = TOL_F32 if dtype == "f32" else TOL_BF16
    assert rowwise_err(out.cpu().numpy(), ref["out"]).max() <= tol
    w.release()


@pytest.mark.parametrize("F", [192, 256, 320, 384, 448, 512])
def test_ffn_widths_cover_each_w2_kernel(gpu_device, F):
    # F / 64 k stages of w2: 3..7 select the register-resident kernel (4..7
    # with stores spread over the next column block), 8 the streamed one
    note(f"bf16 T=700 H=512 E=16 F={F}: every w2 kernel shape vs the oracle")
    inp = synth.make_moe_inputs(T=700, H=512, E=16, F=F, dtype="bf16", seed=40 + F)
    w = weights_for(inp, gpu_device)
    x, gate = x_for(inp, gpu_device), torch.from_numpy(inp.gate).to(gpu_device)
    out = moe.moe_forward_gpu(x, gate, w, out_dtype=torch.float32)
    plan = w.plan_views(inp.T)
    torch.cuda.synchronize()
    ref = oracle.reference_path(inp.x, inp.gate, inp.w1, inp.w3, inp.w2)
    check_plan(plan, ref, inp.T)
    assert rowwise_err(bf16_to_np(plan["y"]), ref["y"]).max() <= TOL_BF16
    assert rowwise_err(out.cpu().numpy(), ref["out"]).max() <= TOL_BF16
    w.release()


def test_empty_batch(gpu_device):
    note("T=0")
    inp = synth.make_moe_inputs(T=0, H=256, E=16, F=64, dtype="bf16", seed=1)
    w = weights_for(inp, gpu_device)
    x = torch.empty((0, 256), dtype=torch.bfloat16, device=gpu_device)
    gate = torch.from_numpy(inp.gate).to(gpu_device)
    out = moe.moe_forward_gpu(x, gate, w)
    torch.cuda.synchronize()
    assert out.shape == (0, 256)
    counts, offsets, arows, rpos = moe.dispatch(torch.empty((0, 2), dtype=torch.uint8, device=gpu_device), 16)
    torch.cuda.synchronize()
    assert counts.abs().sum().item() == 0 and offsets.abs().sum().item() == 0
    w.release()


def test_all_tokens_tie_to_two_experts(gpu_device):
    note("all logits 0: every token -> experts (0, 1); one expert owns every row")
    inp = synth.make_moe_inputs(T=700, H=512, E=16, F=128, dtype="bf16", seed=5)
    inp.gate[:] = 0.0
    w = weights_for(inp, gpu_device)
    x, gate = x_for(inp, gpu_device), torch.from_numpy(inp.gate).to(gpu_device)
    out = moe.moe_forward_gpu(x, gate, w, out_dtype=torch.float32)
    plan = w.plan_views(inp.T)
    torch.cuda.synchronize()
    ref = oracle.reference_path(inp.x, inp.gate, inp.w1, inp.w3, inp.w2)
    assert (ref["routes"] == np.array([0, 1])).all()
    check_plan(plan, ref, inp.T)
    assert rowwise_err(out.cpu().numpy(), ref["out"]).max() <= TOL_BF16
    w.release()


def test_fp32_source_weights_convert_like_bf16_source(gpu_device):
    note("register fp32 weights for bf16 compute == register bf16 weights")
    inp = synth.make_moe_inputs(T=200, H=512, E=8, F=128, dtype="bf16", seed=9)
    w_b = weights_for(inp, gpu_device, src="bf16")
    w_f = weights_for(inp, gpu_device, src="f32", compute=torch.bfloat16)
    x, gate = x_for(inp, gpu_device), torch.from_numpy(inp.gate).to(gpu_device)
    a = moe.moe_forward_gpu(x, gate, w_b)
    b = moe.moe_forward_gpu(x, gate, w_f)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    w_b.release()
    w_f.release()


def test_argument_errors_on_device(gpu_device):
    note("error paths with live weights")
    inp = synth.make_moe_inputs(T=16, H=256, E=16, F=64, dtype="bf16", seed=2)
    w = weights_for(inp, gpu_device)
    gate = torch.from_numpy(inp.gate).to(gpu_device)
    xh = torch.zeros((16, 256), dtype=torch.float16, device=gpu_device)
    with pytest.raises(ValueError):
        moe.moe_forward_gpu(xh, gate, w)           # x dtype does not match bf16 weights
    x = x_for(inp, gpu_device)
    out = torch.empty((16, 256), dtype=torch.bfloat16, device=gpu_device)
    L = capi.lib()
    rc = L.aps_moe_forward(w.handle, x.data_ptr(), capi.DTYPE_BF16, gate.data_ptr(), 16, out.data_ptr(),
                           capi.DTYPE_BF16, 0, 0, None)
    assert rc == capi.APS_ERR_WORKSPACE
    w.release()
    with pytest.raises(ValueError):
        moe.moe_forward_gpu(x, gate, w)            # released handle
