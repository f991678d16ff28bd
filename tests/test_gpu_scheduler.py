"""GPU tests of the w1||w3 GEMM's per-expert tile scheduler (k_ffn_up).

The kernel deals its base list of pieces (wide W: 128 positions x 2 column
blocks, tall T: 256 x 1, S: 128 x 1 for groups of at most 128 positions)
to a persistent grid in rounds and splits the last round's pieces into S or
Q (128 x 1/2) pieces.  These tests drive the staged entry point
aps_moe_ffn_up with synthetic routing plans whose piece counts cover every
branch of that schedule: a handful of pieces (split by 4), about a hundred
(split by 2), just under, at and just over one round (256 CUs), and two
rounds with and without a split tail.  For each plan:
  * the act buffer is poisoned with NaN first, so a position or column the
    schedule misses fails the check;
  * every act row is within 2e-2 (normwise) of the oracle's fp32 SwiGLU
    activations on the same bf16 values;
  * batch independence, bit for bit: each expert's rows computed alone (a
    plan with only that expert, whose few pieces the schedule splits into
    Q pieces) equal its rows in the full plan (W/T/S pieces);
  * a second call gives the same bits.
"""
import sys

import numpy as np
import pytest
import torch

import oracle
from aps2026_amd import capi, moe, synth

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2
F = 448          # 7 column blocks of 64: 3 W pairs + 1 T per 256-position group
E = 16


def note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def base_pieces(counts, nblk=F // 64):
    """Length of the scheduler's base list for per-expert position counts."""
    c = np.asarray(counts, np.int64)
    return int(((nblk // 2) * ((c + 127) // 128) + (nblk & 1) * ((c + 255) // 256)).sum())


def counts_for(target, rng, skew=1.0):
    """Per-expert counts (16 experts) whose base list has about `target`
    pieces: Dirichlet shares, total assignments bisected."""
    p = rng.dirichlet(np.full(E, skew))
    lo, hi = 1, 400000
    while lo < hi:
        mid = (lo + hi) // 2
        if base_pieces(rng_counts(mid, p)) < target:
            lo = mid + 1
        else:
            hi = mid
    return rng_counts(lo, p)


def rng_counts(A, p):
    c = np.floor(p * A).astype(np.int64)
    c[0] += A - c.sum()
    return c


def to_dev_bf16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(torch.bfloat16)


def bf16_bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.fixture(scope="module")
def weights_512(gpu_device):
    inp = synth.make_moe_inputs(T=1024, H=512, E=E, F=F, dtype="bf16", seed=77)
    lists = [[to_dev_bf16(inp.packed[nm + "_bf16"][e], gpu_device) for e in range(E)]
             for nm in ("w1", "w2", "w3")]
    w = moe.register_moe_weights_gpu(lists[0], lists[1], lists[2], compute_dtype=torch.bfloat16)
    yield inp, w
    w.release()


def run_up(w, x, offsets, arows, A, dev):
    act = torch.full((max(A, 1), F), float("nan"), dtype=torch.bfloat16, device=dev)
    off_d = torch.from_numpy(offsets.astype(np.int32)).to(dev)
    rows_d = torch.from_numpy(arows.astype(np.int32)).to(dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = capi.lib().aps_moe_ffn_up(w.handle, x.data_ptr(), capi.DTYPE_BF16, x.shape[0], off_d.data_ptr(),
                                   rows_d.data_ptr(), act.data_ptr(), None, stream)
    assert rc == 0, capi.last_error()
    torch.cuda.synchronize()
    return bf16_bits(act[:A])


def check_plan(inp, w, counts, rng, dev, T=2048):
    A = int(counts.sum())
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.uint32)
    arows = rng.integers(0, T, A).astype(np.uint32)
    xin = synth.make_moe_inputs(T=T, H=inp.H, E=1, F=8, dtype="bf16", seed=int(rng.integers(1 << 30)))
    x = to_dev_bf16(xin.packed["x_bf16"], dev)
    got = run_up(w, x, offsets, arows, A, dev)
    assert np.array_equal(got, run_up(w, x, offsets, arows, A, dev)), "second call differs"
    act = synth.bf16_bits_to_f32(got)
    assert np.isfinite(act).all(), "positions or columns left unwritten"
    experts = np.repeat(np.arange(E, dtype=np.int32), counts)
    _, ref = oracle.ffn_rows(xin.x[arows.astype(np.int64)], experts, inp.w1, inp.w3, inp.w2, want_act=True)
    num = np.linalg.norm(act.astype(np.float64) - ref, axis=1)
    den = np.maximum(np.linalg.norm(ref.astype(np.float64), axis=1), 1e-30)
    assert (num / den).max() <= TOL_BF16
    # each expert alone: its few pieces are split differently, the bits may not change
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi == lo:
            continue
        off_e = np.zeros(E + 1, np.uint32)
        off_e[e + 1:] = hi - lo
        alone = run_up(w, x, off_e, arows[lo:hi], hi - lo, dev)
        assert np.array_equal(alone, got[lo:hi]), f"expert {e}: rows alone differ from the full plan"
    return A


@pytest.mark.parametrize("target", [1, 40, 100, 200, 255, 256, 257, 300, 520, 700])
def test_schedule_covers_every_piece_count(gpu_device, weights_512, target):
    inp, w = weights_512
    rng = np.random.default_rng(1000 + target)
    counts = counts_for(target, rng)
    note(f"up scheduler: target {target} pieces, got {base_pieces(counts)}, counts {counts.tolist()}")
    check_plan(inp, w, counts, rng, gpu_device)


def test_schedule_skewed_and_empty_experts(gpu_device, weights_512):
    inp, w = weights_512
    rng = np.random.default_rng(5)
    counts = np.zeros(E, np.int64)
    counts[[0, 3, 15]] = [9000, 1, 129]       # one hot expert, a single row, one row past a tile
    note(f"up scheduler: skewed counts {counts.tolist()}, {base_pieces(counts)} pieces")
    check_plan(inp, w, counts, rng, gpu_device)


def test_schedule_one_round_overflow_at_full_hidden(gpu_device):
    """C3's size (4096 tokens, hidden 4096, near-uniform routing) puts the
    list just over one round: 257-300 pieces."""
    rng = np.random.default_rng(11)
    inp = synth.make_moe_inputs(T=64, H=4096, E=E, F=F, dtype="bf16", seed=78)
    lists = [[to_dev_bf16(inp.packed[nm + "_bf16"][e], gpu_device) for e in range(E)]
             for nm in ("w1", "w2", "w3")]
    w = moe.register_moe_weights_gpu(lists[0], lists[1], lists[2], compute_dtype=torch.bfloat16)
    try:
        counts = counts_for(280, rng, skew=50.0)
        t = base_pieces(counts)
        note(f"up scheduler: hidden 4096, {t} pieces, counts {counts.tolist()}")
        assert 257 <= t <= 300
        check_plan(inp, w, counts, rng, gpu_device, T=4096)
    finally:
        w.release()
