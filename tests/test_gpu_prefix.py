"""GPU checks of the prefix-deduplication row (reference
PhiTinyMoEModel::generate, src/model.cu:44-159): the row gather bit for bit
against numpy indexing (vector and scalar kernels, repeated and permuted
indices), and the dedup invariant end to end at the C4 shape -- LayerNorm
and the MoE block on the 10,240 trie-node rows, expanded back through
token_node, equal bit for bit the same ops on all 16,384 token rows."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from aps2026_amd import capi, moe, prefix, synth
from tests.test_prefix import c4_prompts

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[case] {msg}", flush=True)


@pytest.mark.parametrize("h,count,offset", [(4096, 777, 0), (4095, 300, 0), (1, 1000, 0), (5000, 64, 0),
                                             (4096, 100, 1), (12, 3, 0)])
def test_gather_rows_bit_exact(gpu_device, h, count, offset):
    note(f"gather h={h} count={count} offset={offset}")
    rng = np.random.default_rng(h + count)
    n = 513
    x = rng.standard_normal((n, h)).astype(np.float32)
    rows = rng.integers(0, n, count)
    rows[:3] = [n - 1, 0, n - 1]
    xd = torch.from_numpy(x).to(gpu_device)
    buf = torch.empty(count * h + offset, dtype=torch.float32, device=gpu_device)
    out = buf[offset:]  # offset 1: unaligned, the scalar kernel
    prefix.gather_rows_gpu(xd, rows, out)
    rib = prefix.RowIndexBuffer(rows, gpu_device)
    out2 = torch.empty((count, h), dtype=torch.float32, device=gpu_device)
    prefix.gather_rows_gpu(xd, rib, out2)
    torch.cuda.synchronize()
    want = oracle.gather_rows(x, rows)
    np.testing.assert_array_equal(out.cpu().numpy().reshape(count, h).view(np.uint32), want.view(np.uint32))
    np.testing.assert_array_equal(out2.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_gather_rows_index_checks(gpu_device):
    x = torch.ones((8, 64), dtype=torch.float32, device=gpu_device)
    out = torch.full((2, 64), 5.0, dtype=torch.float32, device=gpu_device)
    with pytest.raises(ValueError, match="row index"):
        prefix.gather_rows_gpu(x, [1, 8], out)
    # through the C ABI an index past the end gives a zero row, never a read out of bounds
    rows = torch.tensor([3, 8], dtype=torch.int32, device=gpu_device)
    rc = capi.lib().aps_gather_rows(ctypes.c_void_p(x.data_ptr()), 8, 64, ctypes.c_void_p(rows.data_ptr()), 2,
                                    ctypes.c_void_p(out.data_ptr()), None)
    torch.cuda.synchronize()
    assert rc == 0
    assert torch.equal(out[0], torch.ones(64, device=gpu_device))
    assert torch.equal(out[1], torch.zeros(64, device=gpu_device))


def _ancestor_batches():
    rng = np.random.default_rng(11)
    yield "c4", c4_prompts()
    yield "single", [rng.integers(0, 32064, 700).tolist()]
    yield "identical", [[5] * 64] * 6
    yield "tiny-vocab", [rng.integers(0, 3, rng.integers(1, 90)).tolist() for _ in range(40)]
    yield "varied", [rng.integers(0, 40, rng.integers(1, 300)).tolist() for _ in range(25)]
    yield "nested", [[9] * k for k in (1, 200, 3, 64, 4096)]


@pytest.mark.parametrize("name,batch", list(_ancestor_batches()), ids=lambda v: v if isinstance(v, str) else "")
def test_ancestors_gpu_equal_host_table(gpu_device, name, batch):
    """aps_prefix_ancestors builds [nodes][max_len] on the device bit for bit
    equal to the host table (reference src/model.cu:107-116), zero padding
    past each node's depth included."""
    plan = prefix.prefix_dedup(batch)
    note(f"ancestors {name}: {plan.nodes} nodes, stride {plan.max_len}")
    anc = prefix.ancestors_gpu(plan, gpu_device)
    torch.cuda.synchronize()
    assert tuple(anc.shape) == plan.node_anc.shape
    np.testing.assert_array_equal(anc.cpu().numpy().view(np.uint32), plan.node_anc)


def test_ancestors_gpu_argument_checks(gpu_device):
    d = torch.zeros(4, dtype=torch.int32, device=gpu_device)
    lib = capi.lib()
    p = ctypes.c_void_p(d.data_ptr())
    assert lib.aps_prefix_ancestors(p, p, p, 4, 0, p, None) != 0
    assert lib.aps_prefix_ancestors(p, p, p, -1, 4, p, None) != 0
    assert lib.aps_prefix_ancestors(None, p, p, 4, 1, p, None) != 0
    assert lib.aps_prefix_ancestors(None, None, None, 0, 1, None, None) == 0


def test_c4_dedup_rows_equal_full_rows(gpu_device):
    """The invariant the reference's dedup rests on (src/model.cu:64-69), on
    this build's row-wise ops: embedding rows gathered per trie node, then
    LayerNorm and the bf16 MoE block, give bit for bit the rows of the same
    ops run on every packed token row."""
    H, V = 4096, prefix.VOCAB_SIZE
    batch = c4_prompts()
    plan = prefix.prefix_dedup(batch, with_ancestors=False)
    note(f"C4 dedup {plan.token_node.shape[0]} rows -> {plan.nodes} nodes")
    assert plan.nodes == 10240
    g = torch.Generator(device=gpu_device).manual_seed(4)
    emb = torch.randn((V, H), generator=g, device=gpu_device)
    ln_w = 1.0 + 0.05 * torch.randn(H, generator=g, device=gpu_device)
    ln_b = 0.05 * torch.randn(H, generator=g, device=gpu_device)
    ids = np.concatenate([np.asarray(s) for s in batch])
    node_rows = torch.empty((plan.nodes, H), dtype=torch.float32, device=gpu_device)
    full_rows = torch.empty((ids.shape[0], H), dtype=torch.float32, device=gpu_device)
    prefix.gather_rows_gpu(emb, plan.node_token, node_rows)
    prefix.gather_rows_gpu(emb, ids, full_rows)
    tn = torch.from_numpy(plan.token_node.astype(np.int64)).to(gpu_device)
    assert torch.equal(node_rows[tn], full_rows)
    inp = synth.make_moe_inputs(T=16, H=H, E=16, F=448, dtype="bf16", seed=5)
    lists = []
    for nm in ("w1", "w2", "w3"):
        t = torch.from_numpy(np.ascontiguousarray(inp.packed[nm + "_bf16"]).view(np.int16)).to(gpu_device)
        lists.append([t.view(torch.bfloat16)[e].contiguous() for e in range(16)])
    w = moe.register_moe_weights_gpu(*lists, compute_dtype=torch.bfloat16)
    gate = torch.from_numpy(inp.gate).to(gpu_device)
    outs = []
    for rows in (node_rows, full_rows):
        normed = torch.empty_like(rows)
        moe.layer_norm_gpu(rows, ln_w, ln_b, moe.NORM_EPS, normed)
        outs.append(moe.moe_forward_gpu(normed, gate, w, out_dtype=torch.float32))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][tn].view(torch.int32), outs[1].view(torch.int32))
    assert torch.isfinite(outs[1]).all()
    w.release()
