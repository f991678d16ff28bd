"""GPU parity of the tree attention row (reference apply_rope_tree_gpu and
attention_tree_gpu, src/tensor.cu:3342-3377): RoPE and attention through the
C ABI against the oracle bit for bit on prefix-trie batches (the reference's
16 query / 4 KV heads, head_dim 128), with the sliding window exercised at
its real size by a 2,100-token sequence and at a small size; node rows
against token rows; the GQA-4 error."""
import numpy as np
import pytest
import torch

import oracle
from aps2026_amd import attention, prefix
from tests.test_attention import trie_inputs

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[case] {msg}", flush=True)


def dev(a, d):
    return torch.from_numpy(np.ascontiguousarray(a)).to(d)


def shared_batch(seed, groups=3, per=3, pre=40, suf=30):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(groups):
        p = rng.integers(0, 32064, pre).tolist()
        for _ in range(per):
            out.append(p + rng.integers(0, 32064, rng.integers(1, suf)).tolist())
    return out


def test_rope_bit_exact(gpu_device):
    note("rope tree")
    batch = shared_batch(1) + [list(range(1, 300))]
    plan, q, k, _ = trie_inputs(batch, q_heads=16, kv_heads=4, seed=1)
    qd, kd = dev(q, gpu_device), dev(k, gpu_device)
    attention.apply_rope_tree_gpu(qd, kd, plan.node_depth, max_seq=4096)
    torch.cuda.synchronize()
    c, s = oracle.rope_table(4096, 128)
    np.testing.assert_array_equal(qd.cpu().numpy().view(np.uint32),
                                  oracle.rope_tree(q, plan.node_depth, 16, 128, c, s).view(np.uint32))
    np.testing.assert_array_equal(kd.cpu().numpy().view(np.uint32),
                                  oracle.rope_tree(k, plan.node_depth, 4, 128, c, s).view(np.uint32))


@pytest.mark.parametrize("window", [2047, 5])
def test_attention_bit_exact(gpu_device, window):
    note(f"attention tree window={window}")
    batch = shared_batch(2 + window)
    plan, q, k, v = trie_inputs(batch, q_heads=16, kv_heads=4, seed=window)
    out = torch.empty((plan.nodes, 16 * 128), dtype=torch.float32, device=gpu_device)
    attention.attention_tree_gpu(dev(q, gpu_device), dev(k, gpu_device), dev(v, gpu_device), out,
                                 plan.node_depth, plan.node_anc, plan.max_len, window=window)
    torch.cuda.synchronize()
    want = oracle.attention_tree(q, k, v, plan.node_depth, plan.node_anc, plan.max_len, 16, 4, 128, window)
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_attention_long_sequence_sliding_window(gpu_device):
    """One 2,100-token prompt: rows past position 2046 see exactly the last
    2,047 keys (the reference's SLIDING_WINDOW)."""
    note("attention tree 2100-token sequence")
    batch = [list(np.random.default_rng(3).integers(0, 32064, 2100))]
    plan, q, k, v = trie_inputs(batch, q_heads=4, kv_heads=1, seed=3)
    rows = np.arange(plan.nodes - 64, plan.nodes)   # the last 64 rows: full windows
    out = torch.empty((plan.nodes, 4 * 128), dtype=torch.float32, device=gpu_device)
    attention.attention_tree_gpu(dev(q, gpu_device), dev(k, gpu_device), dev(v, gpu_device), out,
                                 plan.node_depth, plan.node_anc, plan.max_len, q_heads=4, kv_heads=1)
    torch.cuda.synchronize()
    want = oracle.attention_tree(q[rows], k, v, plan.node_depth[rows], plan.node_anc[rows], plan.max_len, 4, 1, 128)
    np.testing.assert_array_equal(out.cpu().numpy()[rows].view(np.uint32), want.view(np.uint32))


def test_attention_window_past_64k_of_lds(gpu_device):
    """A 3,500-key window (70 KB of the workgroup's dynamic LDS, past the
    64 KB default) on a 3,500-token prompt: the last rows equal the oracle;
    a window past the LDS budget (7,936 keys) is a shape error."""
    note("attention tree 3500-key window")
    batch = [list(np.random.default_rng(8).integers(0, 32064, 3500))]
    plan, q, k, v = trie_inputs(batch, q_heads=4, kv_heads=1, seed=8)
    rows = np.arange(plan.nodes - 16, plan.nodes)
    out = torch.empty((plan.nodes, 4 * 128), dtype=torch.float32, device=gpu_device)
    attention.attention_tree_gpu(dev(q, gpu_device), dev(k, gpu_device), dev(v, gpu_device), out,
                                 plan.node_depth, plan.node_anc, plan.max_len, q_heads=4, kv_heads=1, window=4096)
    torch.cuda.synchronize()
    want = oracle.attention_tree(q[rows], k, v, plan.node_depth[rows], plan.node_anc[rows], plan.max_len, 4, 1, 128,
                                 4096)
    np.testing.assert_array_equal(out.cpu().numpy()[rows].view(np.uint32), want.view(np.uint32))
    note("attention tree window past the LDS budget")
    q1 = torch.zeros((1, 4 * 128), dtype=torch.float32, device=gpu_device)
    kv1 = torch.zeros((1, 128), dtype=torch.float32, device=gpu_device)
    with pytest.raises(ValueError, match="exceeds"):
        attention.attention_tree_gpu(q1, kv1, kv1, q1.clone(), [0], np.zeros((1, 8000), np.uint32), 8000,
                                     q_heads=4, kv_heads=1, window=8000)


@pytest.mark.parametrize("window", [2047, 300])
def test_attention_long_branches_bit_exact(gpu_device, window):
    """Three 900..1000-token prompts sharing a 600-token prefix: every row,
    with windows longer than and shorter than the chains (keys in many
    64-key chunks, window starts inside a chunk)."""
    note(f"attention tree long branches window={window}")
    rng = np.random.default_rng(window)
    pre = rng.integers(0, 32064, 600).tolist()
    batch = [pre + rng.integers(0, 32064, int(n)).tolist() for n in (300, 350, 400)]
    plan, q, k, v = trie_inputs(batch, q_heads=16, kv_heads=4, seed=window + 1)
    out = torch.empty((plan.nodes, 16 * 128), dtype=torch.float32, device=gpu_device)
    attention.attention_tree_gpu(dev(q, gpu_device), dev(k, gpu_device), dev(v, gpu_device), out,
                                 plan.node_depth, plan.node_anc, plan.max_len, window=window)
    torch.cuda.synchronize()
    want = oracle.attention_tree(q, k, v, plan.node_depth, plan.node_anc, plan.max_len, 16, 4, 128, window)
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("window", [2047, 20])
def test_attention_spread_positions_bit_exact(gpu_device, window):
    """One 300-node chain whose rows are numbered in random order: groups of
    four consecutive rows lie on one chain at scattered positions, in and out
    of order, some further apart than a window (the matrix-core group path and
    the row path both serve such groups)."""
    note(f"attention tree scattered chain positions window={window}")
    n = 300
    rng = np.random.default_rng(11)
    order = rng.permutation(n)                 # order[p] = row at chain position p
    pos = np.empty(n, np.uint32)
    pos[order] = np.arange(n, dtype=np.uint32)
    anc = np.zeros((n, n), np.uint32)
    for r in range(n):
        anc[r, :pos[r] + 1] = order[:pos[r] + 1]
    q = rng.standard_normal((n, 16 * 128)).astype(np.float32)
    k = rng.standard_normal((n, 4 * 128)).astype(np.float32)
    v = rng.standard_normal((n, 4 * 128)).astype(np.float32)
    out = torch.empty((n, 16 * 128), dtype=torch.float32, device=gpu_device)
    attention.attention_tree_gpu(dev(q, gpu_device), dev(k, gpu_device), dev(v, gpu_device), out, pos, anc, n,
                                 window=window)
    torch.cuda.synchronize()
    want = oracle.attention_tree(q, k, v, pos, anc, n, 16, 4, 128, window)
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("window", [2047, 100])
def test_attention_packed_long_sequences_bit_exact(gpu_device, window):
    """aps_attention_packed (the reference's attention_gpu over packed
    sequences) on sequences of 700, 333, 64, 5 and 1 tokens: every row
    against the oracle's attention over its sequence's prefix, bit for bit
    (the packed path-group kernel and the row kernel for rows whose group
    crosses a sequence boundary)."""
    from aps2026_amd import capi
    from aps2026_amd.moe import _ptr, _stream
    note(f"attention packed long sequences window={window}")
    lens = [700, 333, 64, 5, 1]
    rows, stride = sum(lens), max(lens)
    off = np.repeat(np.cumsum([0] + lens[:-1]), lens).astype(np.uint32)
    pos = np.concatenate([np.arange(n) for n in lens]).astype(np.uint32)
    anc = np.zeros((rows, stride), np.uint32)
    for r in range(rows):
        anc[r, :pos[r] + 1] = off[r] + np.arange(pos[r] + 1)
    rng = np.random.default_rng(window)
    q = rng.standard_normal((rows, 16 * 128)).astype(np.float32)
    k = rng.standard_normal((rows, 4 * 128)).astype(np.float32)
    v = rng.standard_normal((rows, 4 * 128)).astype(np.float32)
    qd, kd, vd = dev(q, gpu_device), dev(k, gpu_device), dev(v, gpu_device)
    out = torch.empty((rows, 16 * 128), dtype=torch.float32, device=gpu_device)
    od, pd = dev(off.view(np.int32), gpu_device), dev(pos.view(np.int32), gpu_device)
    rc = capi.lib().aps_attention_packed(_ptr(qd), _ptr(kd), _ptr(vd), _ptr(out), _ptr(od), _ptr(pd), stride, rows,
                                         16, 4, 128, window, _stream(qd.device))
    assert rc == 0, capi.last_error()
    torch.cuda.synchronize()
    want = oracle.attention_tree(q, k, v, pos, anc, stride, 16, 4, 128, window)
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("q_heads,kv_heads,hd,window", [(4, 4, 128, 2047), (8, 1, 64, 2047), (6, 3, 80, 5),
                                                        (16, 2, 128, 300), (3, 1, 1, 2047)])
def test_attention_packed_other_head_layouts_bit_exact(gpu_device, q_heads, kv_heads, hd, window):
    """aps_attention_packed for head layouts other than GQA-4 (multi-head,
    multi-query, 2:1 and 8:1 groups; head_dim 1 to 128), the reference's
    generic k_attention: every row against the oracle bit for bit, on
    sequences of 700, 64, 5 and 1 tokens, with infinities in some value rows
    outside every window of 5 keys."""
    from aps2026_amd import capi
    from aps2026_amd.moe import _ptr, _stream
    note(f"attention packed generic q_heads={q_heads} kv_heads={kv_heads} hd={hd} window={window}")
    lens = [700, 64, 5, 1]
    rows, stride = sum(lens), max(lens)
    off = np.repeat(np.cumsum([0] + lens[:-1]), lens).astype(np.uint32)
    pos = np.concatenate([np.arange(n) for n in lens]).astype(np.uint32)
    rng = np.random.default_rng(q_heads * 100 + hd)
    q = rng.standard_normal((rows, q_heads * hd)).astype(np.float32)
    k = rng.standard_normal((rows, kv_heads * hd)).astype(np.float32)
    v = rng.standard_normal((rows, kv_heads * hd)).astype(np.float32)
    if window == 5:
        v[10:20] = np.inf          # rows 10..19 of the first sequence: only rows up to 24 see them
    qd, kd, vd = dev(q, gpu_device), dev(k, gpu_device), dev(v, gpu_device)
    out = torch.full((rows, q_heads * hd), float("nan"), dtype=torch.float32, device=gpu_device)
    od, pd = dev(off.view(np.int32), gpu_device), dev(pos.view(np.int32), gpu_device)
    rc = capi.lib().aps_attention_packed(_ptr(qd), _ptr(kd), _ptr(vd), _ptr(out), _ptr(od), _ptr(pd), stride, rows,
                                         q_heads, kv_heads, hd, window, _stream(qd.device))
    assert rc == 0, capi.last_error()
    torch.cuda.synchronize()
    want = oracle.attention_generic(q, k, v, off, pos, q_heads, kv_heads, hd, window)
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    if window == 5:
        assert np.isfinite(got[25:]).all()


@pytest.mark.parametrize("window", [2047, 5])
def test_attention_excluded_keys_take_no_part(gpu_device, window):
    """Precondition of the path-group kernel: value rows are finite.  A key
    inside a four-row group's span but outside one row's window (a later row
    of the group, causally, or a key past the sliding window) enters that
    row's value MFMAs with p = 0, which leaves its chains unchanged for every
    finite value; the reference's row kernel never reads such keys.  Value
    rows of +-1e30 at every other position (excluded for the earlier rows of
    each group, and for the later ones at window 5) must leave every output
    bit for bit equal to the oracle's, which reads only in-window keys."""
    from aps2026_amd import capi
    from aps2026_amd.moe import _ptr, _stream
    note(f"attention: large finite values in excluded keys, window={window}")
    lens = [300, 77, 8]
    rows, stride = sum(lens), max(lens)
    off = np.repeat(np.cumsum([0] + lens[:-1]), lens).astype(np.uint32)
    pos = np.concatenate([np.arange(n) for n in lens]).astype(np.uint32)
    anc = np.zeros((rows, stride), np.uint32)
    for r in range(rows):
        anc[r, :pos[r] + 1] = off[r] + np.arange(pos[r] + 1)
    rng = np.random.default_rng(100 + window)
    q = rng.standard_normal((rows, 16 * 128)).astype(np.float32)
    k = rng.standard_normal((rows, 4 * 128)).astype(np.float32)
    v = rng.standard_normal((rows, 4 * 128)).astype(np.float32)
    v[1::2] = np.where(rng.random((v[1::2].shape)) < 0.5, -1e30, 1e30).astype(np.float32)
    qd, kd, vd = dev(q, gpu_device), dev(k, gpu_device), dev(v, gpu_device)
    out = torch.empty((rows, 16 * 128), dtype=torch.float32, device=gpu_device)
    od, pd = dev(off.view(np.int32), gpu_device), dev(pos.view(np.int32), gpu_device)
    rc = capi.lib().aps_attention_packed(_ptr(qd), _ptr(kd), _ptr(vd), _ptr(out), _ptr(od), _ptr(pd), stride, rows,
                                         16, 4, 128, window, _stream(qd.device))
    assert rc == 0, capi.last_error()
    torch.cuda.synchronize()
    want = oracle.attention_tree(q, k, v, pos, anc, stride, 16, 4, 128, window)
    got = out.cpu().numpy()
    assert np.isfinite(got).all() and np.isfinite(want).all()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_attention_nodes_equal_token_rows(gpu_device):
    note("attention tree nodes vs token rows")
    batch = shared_batch(4, groups=2, per=4, pre=60, suf=20)
    plan, q, k, v = trie_inputs(batch, q_heads=16, kv_heads=4, seed=4)
    tn = plan.token_node.astype(np.int64)
    total = tn.shape[0]
    tanc = np.zeros((total, plan.max_len), np.uint32)
    tpos = np.zeros(total, np.uint32)
    for off, ln in zip(plan.offsets, plan.seq_lens):
        for si in range(ln):
            tpos[off + si] = si
            tanc[off + si, :si + 1] = np.arange(off, off + si + 1)
    o_nodes = torch.empty((plan.nodes, 16 * 128), dtype=torch.float32, device=gpu_device)
    o_toks = torch.empty((total, 16 * 128), dtype=torch.float32, device=gpu_device)
    attention.attention_tree_gpu(dev(q, gpu_device), dev(k, gpu_device), dev(v, gpu_device), o_nodes,
                                 plan.node_depth, plan.node_anc, plan.max_len)
    attention.attention_tree_gpu(dev(q[tn], gpu_device), dev(k[tn], gpu_device), dev(v[tn], gpu_device), o_toks,
                                 tpos, tanc, plan.max_len)
    torch.cuda.synchronize()
    assert torch.equal(o_toks.view(torch.int32), o_nodes[torch.from_numpy(tn).to(gpu_device)].view(torch.int32))


def test_attention_errors(gpu_device):
    x = torch.zeros((2, 5 * 128), dtype=torch.float32, device=gpu_device)
    kv = torch.zeros((2, 128), dtype=torch.float32, device=gpu_device)
    with pytest.raises(ValueError, match="expects GQA-4"):
        attention.attention_tree_gpu(x, kv, kv, x.clone(), [0, 1], np.array([[0, 0], [0, 1]]), 2, q_heads=5,
                                     kv_heads=1)
    q = torch.zeros((2, 4 * 128), dtype=torch.float32, device=gpu_device)
    with pytest.raises(ValueError, match="ancestor index"):
        attention.attention_tree_gpu(q, kv, kv, q.clone(), [0, 1], np.array([[0, 0], [0, 7]]), 2, q_heads=4,
                                     kv_heads=1)


@pytest.mark.parametrize("rows,k,n,bias", [(10240 // 40, 4096, 2048, True), (300, 4096, 512, True),
                                           (77, 2048, 4096, True), (64, 256, 12, False), (1, 16, 4, True),
                                           (129, 96, 132, True), (5, 32, 256, False), (200, 48, 20, True),
                                           (2048, 256, 4096, True)])
def test_linear_bit_exact(gpu_device, rows, k, n, bias):
    """aps_linear (the q/k/v/o projections) against the oracle's linear
    (one FMA chain per output, k ascending, then the bias), bit for bit."""
    note(f"linear rows={rows} k={k} n={n} bias={bias}")
    rng = np.random.default_rng(rows + k + n)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    w = (0.02 * rng.standard_normal((n, k))).astype(np.float32)
    b = (0.1 * rng.standard_normal(n)).astype(np.float32) if bias else None
    got = attention.linear_gpu(dev(x, gpu_device), dev(w, gpu_device), dev(b, gpu_device) if bias else None)
    torch.cuda.synchronize()
    want = oracle.linear(x, w, b)
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows,k,n,bias,offset", [(13, 37, 5, True, 0), (1, 1, 1, False, 0), (70, 17, 131, True, 0),
                                                  (65, 4096, 6, True, 1), (200, 48, 20, True, 1),
                                                  (3, 300, 65, False, 3), (130, 15, 64, True, 0)])
def test_linear_general_shapes_bit_exact(gpu_device, rows, k, n, bias, offset):
    """aps_linear on shapes the vector and matrix-core kernels do not take
    (k % 16 != 0, n % 4 != 0, or arrays 4- but not 16-byte aligned: `offset`
    floats into a buffer), the reference's tiled fallback: bit for bit
    against the oracle's chain.  Row 0 of x is zero, so its products are
    zeros of both signs: its sums must come out +0, as the chain gives,
    through the zero-padded k steps too."""
    note(f"linear general rows={rows} k={k} n={n} bias={bias} offset={offset}")
    rng = np.random.default_rng(rows * 7 + k + n)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    w = (0.02 * rng.standard_normal((n, k))).astype(np.float32)
    x[0] = 0.0
    b = (0.1 * rng.standard_normal(n)).astype(np.float32) if bias else None

    def placed(a):
        buf = torch.full((a.size + offset,), float("nan"), dtype=torch.float32, device=gpu_device)
        buf[offset:] = torch.from_numpy(a.ravel()).to(gpu_device)
        return buf[offset:]

    from aps2026_amd import capi
    from aps2026_amd.moe import _ptr, _stream
    xd, wd = placed(x), placed(w)
    bd = placed(b) if bias else None
    y = placed(np.full((rows, n), np.nan, np.float32))
    rc = capi.lib().aps_linear(_ptr(xd), _ptr(wd), _ptr(bd) if bias else None, rows, k, n, _ptr(y),
                               _stream(xd.device))
    assert rc == 0, capi.last_error()
    torch.cuda.synchronize()
    want = oracle.linear(x, w, b)
    np.testing.assert_array_equal(y.cpu().numpy().reshape(rows, n).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows,k,ns,bias", [(10240 // 20, 4096, (512, 512), (True, True)),
                                            (300, 256, (2048, 512, 132), (True, False, True)),
                                            (129, 96, (64, 20), (False, True)), (7, 48, (4, 8, 12), (True, True, True)),
                                            (2048, 256, (4096,), (True,))])
def test_linear_multi_bit_exact(gpu_device, rows, k, ns, bias):
    """aps_linear_multi (k and v of one input in one grid, the reference's
    matmul_pair_bias_gpu) against the oracle's linear per output, bit for
    bit: one and two and three outputs, the 128- and the 64-column block
    grid, outputs of unequal width, k = 48 (the vector-FMA fallback) and
    missing biases."""
    import ctypes
    from aps2026_amd import capi
    from aps2026_amd.moe import _ptr, _stream
    note(f"linear multi rows={rows} k={k} ns={ns}")
    rng = np.random.default_rng(rows + k + sum(ns))
    x = rng.standard_normal((rows, k)).astype(np.float32)
    ws = [(0.02 * rng.standard_normal((n, k))).astype(np.float32) for n in ns]
    bs = [(0.1 * rng.standard_normal(n)).astype(np.float32) if b else None for n, b in zip(ns, bias)]
    xd = dev(x, gpu_device)
    wd = [dev(w, gpu_device) for w in ws]
    bd = [dev(b, gpu_device) if b is not None else None for b in bs]
    ys = [torch.full((rows, n), float("nan"), dtype=torch.float32, device=gpu_device) for n in ns]
    cnt = len(ns)
    vp = ctypes.c_void_p * cnt
    rc = capi.lib().aps_linear_multi(_ptr(xd), rows, k, cnt, vp(*[_ptr(w) for w in wd]), vp(*[_ptr(b) for b in bd]),
                                     (ctypes.c_int32 * cnt)(*ns), vp(*[_ptr(y) for y in ys]), _stream(xd.device))
    assert rc == 0, capi.last_error()
    torch.cuda.synchronize()
    for y, w, b in zip(ys, ws, bs):
        np.testing.assert_array_equal(y.cpu().numpy().view(np.uint32), oracle.linear(x, w, b).view(np.uint32))


def test_linear_bit_exact_wide_exponents(gpu_device):
    """The matrix-core Linear (K = 1 fp32 MFMA chains) against the oracle's
    FMA chain on operands whose exponents span 2^-20 .. 2^20 and on products
    around FLT_MIN, where a product rounded before the add (no fused
    multiply-add) or a flushed subnormal would change bits."""
    rng = np.random.default_rng(3)
    rows, k, n = 130, 512, 160
    for scale in ("spread", "tiny"):
        note(f"linear wide-exponent case {scale}")
        if scale == "spread":
            x = (rng.uniform(-1, 1, (rows, k)) * np.exp2(rng.integers(-20, 20, (rows, k)))).astype(np.float32)
            w = (rng.uniform(-1, 1, (n, k)) * np.exp2(rng.integers(-20, 20, (n, k)))).astype(np.float32)
        else:
            x = (rng.uniform(-1, 1, (rows, k)) * 1e-19).astype(np.float32)
            w = (rng.uniform(-1, 1, (n, k)) * 1e-19).astype(np.float32)
        b = (0.1 * rng.standard_normal(n)).astype(np.float32)
        got = attention.linear_gpu(dev(x, gpu_device), dev(w, gpu_device), dev(b, gpu_device))
        torch.cuda.synchronize()
        want = oracle.linear(x, w, b)
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))
