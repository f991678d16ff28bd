"""The reference's optional tensor-core Linear (USE_TC / USE_TC_ALL: split
bf16 hi/lo products, src/tensor.cu:124-177, 514-584): the oracle's
restatement pinned on the CPU, then the HIP path (aps_linear_tc) against it
on the GPU.  Not bit-exact by design: the tensor cores' accumulation order is
unspecified, so the GPU is held to the fp64 sum of the exact bf16 products
within fp32 accumulation error, and both to the fp32 Linear within the
split's own error."""
import numpy as np
import pytest
import torch

import oracle


def _scale(x, w):
    """sum_k |x_k w_k| per output: the size every rounding error scales with."""
    return np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T


def test_bf16_split_known_answers_and_reconstruction():
    v = np.array([1.0, 1 + 2 ** -10, 1 + 2 ** -8, 1 + 3 * 2 ** -8, -2.5, 3.0e-30, 0.0], np.float32)
    hi, lo = oracle.bf16_split(v)
    # 1 + 2^-10 rounds down to 1 (bf16 keeps 7 fraction bits); 1 + 2^-8 is a tie
    # and goes to the even 1.0; 1 + 3 * 2^-8 rounds up to 1 + 2^-6
    assert hi.tolist()[:5] == [1.0, 1.0, 1.0, 1 + 2 ** -6, -2.5]
    assert lo.tolist()[:5] == [0.0, 2 ** -10, 2 ** -8, -(2 ** -8), 0.0]
    assert (hi.view(np.uint32) & 0xFFFF).max() == 0 and (lo.view(np.uint32) & 0xFFFF).max() == 0
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(100000) * np.exp2(rng.integers(-30, 30, 100000))).astype(np.float32)
    hi, lo = oracle.bf16_split(x)
    err = np.abs(x.astype(np.float64) - hi.astype(np.float64) - lo.astype(np.float64))
    assert np.all(err <= 2.0 ** -16 * np.abs(x))


def test_split_linear_exact_on_bf16_operands():
    """Operands that are bf16 already have lo = 0: the three (four) terms
    reduce to the one exact product, here small integers summed exactly."""
    rng = np.random.default_rng(1)
    x = rng.integers(-8, 8, (5, 64)).astype(np.float32)
    w = rng.integers(-8, 8, (12, 64)).astype(np.float32)
    b = rng.integers(-4, 4, 12).astype(np.float32)
    want = (x.astype(np.int64) @ w.T.astype(np.int64) + b.astype(np.int64)).astype(np.float32)
    for all_terms in (False, True):
        assert np.array_equal(oracle.linear_split_bf16(x, w, b, all_terms), want)
    assert np.array_equal(oracle.linear(x, w, b), want)


def test_split_linear_close_to_fp32_and_a_dropped_term_is_caught():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((16, 512)).astype(np.float32)
    w = (0.02 * rng.standard_normal((24, 512))).astype(np.float32)
    ref = oracle.linear(x, w)
    sc = _scale(x, w)
    e3 = np.abs(oracle.linear_split_bf16(x, w) - ref) / sc
    e4 = np.abs(oracle.linear_split_bf16(x, w, all_terms=True) - ref) / sc
    assert e3.max() < 3e-5 and e4.max() < 2e-6
    # a restatement that forgot x_hi w_lo is off by about 2^-9 of the scale
    xh, xl = oracle.bf16_split(x)
    wh, _ = oracle.bf16_split(w)
    bad = (xh.astype(np.float64) @ wh.T + xl.astype(np.float64) @ wh.T).astype(np.float32)
    assert (np.abs(bad - ref) / sc).max() > 3e-5


@pytest.mark.gpu
@pytest.mark.parametrize("rows,k,n,all_terms", [(300, 4096, 512, False), (300, 4096, 512, True),
                                                (4096, 2048, 4096, False), (77, 64, 100, True),
                                                (129, 256, 2052, False)])
def test_linear_tc_gpu_matches_the_split_products(gpu_device, rows, k, n, all_terms):
    from aps2026_amd import attention
    print(f"[case] linear tc rows={rows} k={k} n={n} all={all_terms}", flush=True)
    rng = np.random.default_rng(rows + n)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    w = (0.02 * rng.standard_normal((n, k))).astype(np.float32)
    b = (0.1 * rng.standard_normal(n)).astype(np.float32)
    xd = torch.from_numpy(x).to(gpu_device)
    packed = attention.linear_tc_prepare(torch.from_numpy(w).to(gpu_device))
    got = attention.linear_tc_gpu(attention.linear_tc_split(xd), packed, n, torch.from_numpy(b).to(gpu_device),
                                  all_terms).cpu().numpy()
    sample = slice(0, min(rows, 256))   # the fp64 references on a row sample at the large shapes
    g = got[sample]
    sc = _scale(x[sample], w)
    emu = oracle.linear_split_bf16(x[sample], w, b, all_terms)
    err_emu = (np.abs(g - emu) / (sc + np.abs(b))).max()
    err_f32 = (np.abs(g - oracle.linear(x[sample], w, b)) / (sc + np.abs(b))).max()
    print(f"[case] max error / scale: vs split products {err_emu:.2e}, vs fp32 Linear {err_f32:.2e}", flush=True)
    assert err_emu < 2e-6
    assert err_f32 < (3e-5 if not all_terms else 5e-6)
    assert np.isfinite(got).all()


@pytest.mark.gpu
def test_linear_tc_multi_equals_single_launches(gpu_device):
    """aps_linear_tc_multi (q, k and v of one split input in one launch)
    equals one aps_linear_tc per output bit for bit."""
    import ctypes
    from aps2026_amd import attention, capi
    from aps2026_amd.moe import _ptr, _stream
    rows, k, ns = 300, 512, (256, 132, 64)
    print(f"[case] linear tc multi rows={rows} k={k} ns={ns}", flush=True)
    rng = np.random.default_rng(4)
    x = torch.from_numpy(rng.standard_normal((rows, k)).astype(np.float32)).to(gpu_device)
    ws = [torch.from_numpy((0.02 * rng.standard_normal((n, k))).astype(np.float32)).to(gpu_device) for n in ns]
    bs = [torch.from_numpy((0.1 * rng.standard_normal(n)).astype(np.float32)).to(gpu_device) for n in ns]
    bs[1] = None
    packed = [attention.linear_tc_prepare(w) for w in ws]
    xs = attention.linear_tc_split(x)
    for all_terms in (False, True):
        want = [attention.linear_tc_gpu(xs, p, n, b, all_terms) for p, n, b in zip(packed, ns, bs)]
        got = [torch.empty_like(w_) for w_ in want]
        vp = ctypes.c_void_p * 3
        rc = capi.lib().aps_linear_tc_multi(_ptr(xs), rows, k, 3, vp(*[_ptr(p) for p in packed]),
                                            vp(*[_ptr(b) for b in bs]), (ctypes.c_int32 * 3)(*ns), int(all_terms),
                                            vp(*[_ptr(g) for g in got]), _stream(x.device))
        assert rc == 0, capi.last_error()
        torch.cuda.synchronize()
        for g, w_ in zip(got, want):
            assert torch.equal(g.view(torch.int32), w_.view(torch.int32))
