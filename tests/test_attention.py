"""Tree attention oracle (scope row f4: reference k_rope and
k_attention_tree_gqa4, src/tensor.cu:2180-2197, 2407-2633, rope_table
:2703-2735) pinned by what the mathematics fixes: identity rotation at
position 0, fp64 rotations and fp64 softmax attention, a single key giving
its value exactly, duplicate keys, the sliding window, and the reference's
own claim that attention on trie nodes equals attention on token rows bit
for bit.  Also the library's host RoPE table against the oracle's."""
import numpy as np
import pytest

import oracle
from aps2026_amd import attention, prefix


def trie_inputs(batch, q_heads=8, kv_heads=2, hd=128, seed=0):
    plan = prefix.prefix_dedup(batch)
    rng = np.random.default_rng(seed)
    n = plan.nodes
    q = rng.standard_normal((n, q_heads * hd)).astype(np.float32)
    k = rng.standard_normal((n, kv_heads * hd)).astype(np.float32)
    v = rng.standard_normal((n, kv_heads * hd)).astype(np.float32)
    return plan, q, k, v


def fp64_attention(q, k, v, pos, anc, q_heads, kv_heads, hd, window):
    out = np.zeros((q.shape[0], q_heads * hd))
    g = q_heads // kv_heads
    for r in range(q.shape[0]):
        p = int(pos[r])
        b = max(0, p + 1 - window)
        keys = anc[r, b:p + 1].astype(np.int64)
        for h in range(q_heads):
            kh = h // g
            qv = q[r, h * hd:(h + 1) * hd].astype(np.float64)
            K = k[keys, kh * hd:(kh + 1) * hd].astype(np.float64)
            V = v[keys, kh * hd:(kh + 1) * hd].astype(np.float64)
            s = K @ qv / np.sqrt(hd)
            e = np.exp(s - s.max())
            out[r, h * hd:(h + 1) * hd] = (e / e.sum()) @ V
    return out


def test_rope_table_pins():
    c, s = oracle.rope_table(4096, 128)
    assert (c[0] == 1).all() and (s[0] == 0).all()
    half = 64
    inv = np.array([np.float32(np.power(np.float64(10000.0), np.float64(np.float32(-2.0 * j) / np.float32(128))))
                    for j in range(half)], np.float64)
    p = np.arange(4096, dtype=np.float64)[:, None]
    ang = (p * inv[None, :]).astype(np.float32).astype(np.float64)   # the float angle
    assert np.abs(c - np.cos(ang)).max() < 1.2e-7 and np.abs(s - np.sin(ang)).max() < 1.2e-7
    assert np.abs(c * c.astype(np.float64) + s * s.astype(np.float64) - 1).max() < 1e-6


def test_library_rope_table_equals_oracle():
    for max_seq, hd, theta in ((4096, 128, 10000.0), (33, 64, 500.0)):
        a = attention.rope_table(max_seq, hd, theta)
        b = oracle.rope_table(max_seq, hd, theta)
        assert all(np.array_equal(x.view(np.uint32), y.view(np.uint32)) for x, y in zip(a, b))


def test_rope_pins():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((6, 3 * 128)).astype(np.float32)
    pos = np.array([0, 1, 7, 100, 2047, 4095], np.uint32)
    c, s = oracle.rope_table(4096, 128)
    y = oracle.rope_tree(x, pos, 3, 128, c, s)
    assert np.array_equal(y[0].view(np.uint32), x[0].view(np.uint32))      # position 0: identity
    xr, yr = x.reshape(6, 3, 2, 64).astype(np.float64), y.reshape(6, 3, 2, 64).astype(np.float64)
    cc, ss = c[pos.astype(np.int64)][:, None, :], s[pos.astype(np.int64)][:, None, :]
    want0 = xr[:, :, 0] * cc - xr[:, :, 1] * ss
    want1 = xr[:, :, 1] * cc + xr[:, :, 0] * ss
    assert np.abs(yr[:, :, 0] - want0).max() < 1e-6 and np.abs(yr[:, :, 1] - want1).max() < 1e-6
    # a plausible mistake -- the halves swapped -- is far off
    assert np.abs(yr[:, :, 1] - (xr[:, :, 1] * cc - xr[:, :, 0] * ss))[1:].max() > 0.1


def test_attention_single_key_is_its_value():
    q = np.random.default_rng(2).standard_normal((1, 4 * 128)).astype(np.float32)
    k = np.random.default_rng(3).standard_normal((1, 128)).astype(np.float32)
    v = np.random.default_rng(4).standard_normal((1, 128)).astype(np.float32)
    out = oracle.attention_tree(q, k, v, np.array([0], np.uint32), np.array([[0]], np.uint32), 1, 4, 1, 128)
    assert np.array_equal(out.reshape(4, 128), np.tile(v, (4, 1)))


def test_attention_duplicate_keys():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((2, 4 * 128)).astype(np.float32)
    k = np.tile(rng.standard_normal((1, 128)).astype(np.float32), (2, 1))
    v = np.tile(rng.standard_normal((1, 128)).astype(np.float32), (2, 1))
    anc = np.array([[0, 0], [0, 1]], np.uint32)
    out = oracle.attention_tree(q, k, v, np.array([0, 1], np.uint32), anc, 2, 4, 1, 128)
    assert np.array_equal(out[1].reshape(4, 128), np.tile(v[0], (4, 1)))   # p = 1/2 each, exactly


@pytest.mark.parametrize("window", [2047, 3])
def test_attention_against_fp64(window):
    batch = [[1, 2, 3, 4, 5, 6, 7], [1, 2, 3, 9, 9], [4, 4], [1, 2, 8, 8, 8, 8, 8, 8, 8, 8]]
    plan, q, k, v = trie_inputs(batch, seed=window)
    out = oracle.attention_tree(q, k, v, plan.node_depth, plan.node_anc, plan.max_len, 8, 2, 128, window)
    want = fp64_attention(q, k, v, plan.node_depth, plan.node_anc, 8, 2, 128, window)
    assert np.abs(out - want).max() < 1e-5 * max(1.0, np.abs(want).max())


def packed_inputs(lens, q_heads, kv_heads, hd, seed):
    """Packed sequences of the given lengths: q, k, v and each row's segment
    start and position."""
    rows = int(sum(lens))
    seg_offset = np.concatenate([np.full(n, int(sum(lens[:i])), np.uint32) for i, n in enumerate(lens)])
    seg_pos = np.concatenate([np.arange(n, dtype=np.uint32) for n in lens])
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((rows, q_heads * hd)).astype(np.float32)
    k = rng.standard_normal((rows, kv_heads * hd)).astype(np.float32)
    v = rng.standard_normal((rows, kv_heads * hd)).astype(np.float32)
    return q, k, v, seg_offset, seg_pos


@pytest.mark.parametrize("q_heads,kv_heads,hd,window", [(4, 4, 64, 2047), (8, 1, 128, 5), (6, 3, 80, 2047),
                                                        (3, 1, 32, 2)])
def test_attention_generic_against_fp64(q_heads, kv_heads, hd, window):
    """The generic-layout attention oracle (reference k_attention) against a
    float64 softmax attention over each row's own sequence prefix: pins the
    head mapping kh = qh / (q_heads / kv_heads), the segment indexing and the
    sliding window (a head or segment mix-up is far off)."""
    lens = [7, 1, 12, 3]
    q, k, v, off, pos = packed_inputs(lens, q_heads, kv_heads, hd, seed=q_heads + hd)
    out = oracle.attention_generic(q, k, v, off, pos, q_heads, kv_heads, hd, window)
    anc = np.zeros((q.shape[0], max(lens)), np.uint32)
    for r in range(q.shape[0]):
        anc[r, :pos[r] + 1] = off[r] + np.arange(pos[r] + 1)
    want = fp64_attention(q, k, v, pos, anc, q_heads, kv_heads, hd, window)
    assert np.abs(out - want).max() < 1e-5 * max(1.0, np.abs(want).max())
    # a plausible mistake -- the keys of the whole packed batch instead of the
    # row's own sequence -- is far off
    anc_all = np.zeros_like(anc)
    for r in range(q.shape[0]):
        b = max(0, r + 1 - max(lens))
        anc_all[r, :min(r + 1, max(lens))] = np.arange(b, r + 1)[-max(lens):]
    wrong = fp64_attention(q, k, v, np.minimum(np.arange(q.shape[0]), max(lens) - 1).astype(np.uint32), anc_all,
                           q_heads, kv_heads, hd, window)
    assert np.abs(out - wrong).max() > 1e-2


def test_attention_generic_closed_forms():
    """Exact cases: a row's first position attends to itself alone (p = 1, out
    = v); with q = 0 every score is 0, e = 1, den = n, so p = RN(1 / n) and
    the output is the fma chain of RN(1 / n) v_w; a value outside the window
    does not reach the row."""
    hd = 48
    q, k, v, off, pos = packed_inputs([5, 3], 2, 2, hd, seed=9)
    out = oracle.attention_generic(q, k, v, off, pos, 2, 2, hd, 2047)
    assert np.array_equal(out[0].view(np.uint32), v[0].view(np.uint32))       # row 0 of sequence 0
    assert np.array_equal(out[5].view(np.uint32), v[5].view(np.uint32))       # row 0 of sequence 1
    qz = np.zeros_like(q)
    out = oracle.attention_generic(qz, k, v, off, pos, 2, 2, hd, 2047)
    r = 4                                                                      # position 4: keys 0..4
    p = np.float32(1.0) / np.float32(5.0)
    want = np.zeros(2 * hd, np.float32)
    for w in range(5):
        want = (np.float64(p) * v[w].astype(np.float64) + want.astype(np.float64)).astype(np.float32)
    assert np.array_equal(out[r].view(np.uint32), want.view(np.uint32))
    vb = v.copy()
    vb[0] = 1e30                                                               # outside row 4's window of 2
    a = oracle.attention_generic(q, k, v, off, pos, 2, 2, hd, 2)
    b = oracle.attention_generic(q, k, vb, off, pos, 2, 2, hd, 2)
    assert np.array_equal(a[2:5].view(np.uint32), b[2:5].view(np.uint32))


def test_attention_generic_scores_are_one_chain_over_d():
    """The generic kernel scores with ONE fma chain over d (reference
    k_attention), not the GQA-4 kernel's four partial sums: with q . k terms
    (1e8, 1, -1e8, 1) the chain gives 1 (1e8 + 1 rounds to 1e8, the
    cancellation leaves the last 1) and the partial sums
    (1e8 + 1) + (-1e8 + 1) give 0.  Row 1 attends to key 0 (that score) and
    key 1 (score 0)."""
    hd = 4
    q = np.zeros((2, hd), np.float32)
    k = np.zeros((2, hd), np.float32)
    q[1] = [1e8, 1.0, -1e8, 1.0]
    k[0] = [1.0, 1.0, 1.0, 1.0]
    v = np.array([[1.0, 0.0, 0.0, 0.0], [0.0, 1.0, 0.0, 0.0]], np.float32)
    out = oracle.attention_generic(q, k, v, np.zeros(2, np.uint32), np.array([0, 1], np.uint32), 1, 1, hd, 2047)
    s0 = 1.0 / np.sqrt(hd)
    p0 = np.exp(s0) / (np.exp(s0) + 1.0)
    assert abs(out[1, 0] - p0) < 1e-6 and abs(out[1, 1] - (1 - p0)) < 1e-6
    assert abs(out[1, 0] - 0.5) > 0.05           # the four-partial score (0) would give 1/2


def test_attention_tree_equals_token_rows():
    """src/layer.cu:181-185: attention on the trie nodes equals attention on
    the packed token rows (each token its own row, its keys the rows of its
    own prefix) bit for bit."""
    rng = np.random.default_rng(7)
    pre = rng.integers(0, 50, 9).tolist()
    batch = [pre + rng.integers(0, 50, 6).tolist(), pre + rng.integers(0, 50, 4).tolist(), pre[:5]]
    plan, q, k, v = trie_inputs(batch, q_heads=4, kv_heads=1, seed=8)
    node_out = oracle.attention_tree(q, k, v, plan.node_depth, plan.node_anc, plan.max_len, 4, 1, 128)
    tn = plan.token_node.astype(np.int64)
    total = tn.shape[0]
    tanc = np.zeros((total, plan.max_len), np.uint32)
    tpos = np.zeros(total, np.uint32)
    for b, (off, ln) in enumerate(zip(plan.offsets, plan.seq_lens)):
        for si in range(ln):
            tpos[off + si] = si
            tanc[off + si, :si + 1] = np.arange(off, off + si + 1)
    tok_out = oracle.attention_tree(q[tn], k[tn], v[tn], tpos, tanc, plan.max_len, 4, 1, 128)
    assert np.array_equal(tok_out.view(np.uint32), node_out[tn].view(np.uint32))


def test_linear_pins():
    """oracle.linear: equals the router-logits chain for narrow outputs (the
    same FMA chain), its bias is one exact fp32 add, and it is within the
    fp64 error bound of the product."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((5, 512)).astype(np.float32)
    w = rng.standard_normal((40, 512)).astype(np.float32)
    b = rng.standard_normal(40).astype(np.float32)
    y0 = oracle.linear(x, w)
    assert np.array_equal(y0.view(np.uint32), oracle.router_logits(x, w).view(np.uint32))
    assert np.array_equal(oracle.linear(x, w, b), (y0 + b).astype(np.float32))
    ref = x.astype(np.float64) @ w.T.astype(np.float64)
    bound = 512 * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(w).T.astype(np.float64))
    assert (np.abs(y0 - ref) <= bound).all()
    wide = rng.standard_normal((300, 512)).astype(np.float32)
    yw = oracle.linear(x, wide)
    assert np.array_equal(yw[:, :40].view(np.uint32), oracle.linear(x, wide[:40]).view(np.uint32))
