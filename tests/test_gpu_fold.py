"""GPU tests of the fp8 path's folded combine (aps_moe_forward with fp8
experts, F in (384, 512], bf16 output).

The dispatch also writes each expert's positions reordered by route slot
(slot1, slot_rows, slot_tokens in the workspace); the w2 GEMM then runs as
two launches over those lists, the first storing each slot-0 row's bf16
output row by token, the second combining each slot-1 row with it into the
output: (0 + 0.5 a) + 0.5 b, the reference's combine.

  * the slot-ordered lists equal a numpy construction from the routing plan,
    and the plan itself (offsets, assignment_rows, route_positions) is the
    reference's, bit for bit against the oracle;
  * the folded output equals the unfolded path's (w2 to y by position, then
    k_combine), bit for bit, over batch sizes that put the w2 GEMM's tiles
    at different column splits, ragged tiles, a batch whose experts see
    routes of one slot only, and repeated calls on one workspace;
  * fp32 output takes the unfolded path: the fused and grouped entry
    points agree bit for bit.
"""
import sys

import numpy as np
import pytest
import torch

import oracle
from aps2026_amd import moe, synth
from tests.test_gpu_fp8 import fp8_weights, to_dev_bf16

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def slot_views(w, rows):
    ws, L = w.workspace(rows)
    E = w.num_experts

    def view(off, n):
        return ws[off:off + 4 * n].view(torch.int32)
    return (view(L.slot1, E).cpu().numpy().view(np.uint32), view(L.slot_rows, 2 * rows).cpu().numpy().view(np.uint32),
            view(L.slot_tokens, 2 * rows).cpu().numpy().view(np.uint32))


def expected_slots(plan, E):
    routes = plan["routes"].cpu().numpy().astype(np.int64)
    offsets = plan["offsets"].cpu().numpy().view(np.uint32).astype(np.int64)
    arows = plan["assignment_rows"].cpu().numpy().view(np.uint32).astype(np.int64)
    slot1 = np.zeros(E, np.uint32)
    srows, stoks = [], []
    for e in range(E):
        p = np.arange(offsets[e], offsets[e + 1])
        t = arows[p]
        first = routes[t, 0] == e
        slot1[e] = offsets[e] + first.sum()
        srows += [p[first], p[~first]]
        stoks += [t[first], t[~first]]
    return slot1, np.concatenate(srows).astype(np.uint32), np.concatenate(stoks).astype(np.uint32)


def run_both(w, x, gate, T):
    out = moe.moe_forward_gpu(x, gate, w, out_dtype=torch.bfloat16)
    plan = w.plan_views(T)
    slots = slot_views(w, T)
    logits = plan["logits"].clone()
    out_g = moe.moe_forward_grouped_gpu(x, logits, w, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    return out, out_g, plan, slots


def check(inp, dev, reps=1):
    w = fp8_weights(inp, dev)
    x = to_dev_bf16(inp.packed["x_bf16"], dev)
    gate = torch.from_numpy(inp.gate).to(dev)
    try:
        for r in range(reps):
            out, out_g, plan, (slot1, srows, stoks) = run_both(w, x, gate, inp.T)
            ref_routes = oracle.route_top2(oracle.router_logits(inp.x, inp.gate))
            counts, offsets, rows, pos = oracle.dispatch(ref_routes, inp.E)
            np.testing.assert_array_equal(plan["routes"].cpu().numpy().astype(np.int32), ref_routes)
            np.testing.assert_array_equal(plan["offsets"].cpu().numpy().view(np.uint32), offsets)
            np.testing.assert_array_equal(plan["assignment_rows"].cpu().numpy().view(np.uint32), rows)
            np.testing.assert_array_equal(plan["route_positions"].cpu().numpy().view(np.uint32), pos)
            e1, er, et = expected_slots(plan, inp.E)
            A = 2 * inp.T
            np.testing.assert_array_equal(slot1, e1)
            np.testing.assert_array_equal(srows[:A], er)
            np.testing.assert_array_equal(stoks[:A], et)
            diff = int((out.view(torch.int16) != out_g.view(torch.int16)).sum())
            assert diff == 0, f"rep {r}: folded combine differs from w2 + combine in {diff} elements"
            assert torch.isfinite(out.float()).all()
    finally:
        w.release()


@pytest.mark.parametrize("T,H", [(1, 1024), (2, 1024), (100, 1024), (333, 2048), (1000, 4096), (4097, 4096),
                                 (12345, 1024)])
def test_fold_equals_w2_and_combine(gpu_device, T, H):
    note(f"folded combine fp8 T={T} H={H} E=16 F=448")
    inp = synth.make_moe_inputs(T=T, H=H, E=16, F=448, dtype="fp8", seed=900 + T, name="fold")
    check(inp, gpu_device)


def test_fold_c5_zipf_repeated(gpu_device):
    """C5 (8192 tokens, Zipf(1.1) expert loads), three calls on one workspace."""
    note("folded combine at C5, three calls")
    check(synth.make_config("c5"), gpu_device, reps=3)


def test_fold_f_widths_and_single_slot_experts(gpu_device):
    """F = 512 (w2's four k stages exactly) folds too; E = 2 puts every
    token's routes on both experts, so each expert sees both slots; E = 3
    with T = 5 leaves experts with routes of one slot only."""
    for T, H, E, F in ((700, 1024, 16, 512), (500, 1024, 2, 448), (5, 1024, 3, 448)):
        note(f"folded combine fp8 T={T} H={H} E={E} F={F}")
        inp = synth.make_moe_inputs(T=T, H=H, E=E, F=F, dtype="fp8", seed=77 + T + E, name="fold-w")
        check(inp, gpu_device)


def test_fp32_output_takes_the_unfolded_path(gpu_device):
    inp = synth.make_moe_inputs(T=300, H=1024, E=16, F=448, dtype="fp8", seed=5, name="fold-f32")
    w = fp8_weights(inp, gpu_device)
    x = to_dev_bf16(inp.packed["x_bf16"], gpu_device)
    gate = torch.from_numpy(inp.gate).to(gpu_device)
    try:
        a = moe.moe_forward_gpu(x, gate, w, out_dtype=torch.float32)
        logits = w.plan_views(inp.T)["logits"].clone()
        b = moe.moe_forward_grouped_gpu(x, logits, w, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    finally:
        w.release()
