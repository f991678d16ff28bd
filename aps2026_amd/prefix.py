"""Prompt prefix deduplication and the row gather it feeds, over the C ABI
(include/aps_moe.h).

Reference API mirrored (file:line in the reference tree):
  PhiTinyMoEModel::generate prefix trie   src/model.cu:44-117
  tensor_ops::gather_rows_gpu             include/tensor.h:115-116, 138
  tensor_ops::RowIndexBuffer              include/tensor.h:119-137

A token's hidden state depends only on the prefix that ends at it (causal
attention, independent sequences), so every row-wise op of a layer runs on
the nodes of the prompts' prefix trie: ``prefix_dedup`` builds the trie
(host code in libaps_moe.so, the reference's node numbering), and
``gather_rows_gpu`` copies embedding rows to node rows (and, at the end,
the last token of each prompt) with the HIP gather kernel.

Errors: the reference's std::invalid_argument conditions raise ValueError
with its messages ("empty input", "sequence is too long", "token out of
vocabulary"); an empty batch raises RuntimeError("generate received an
empty input batch") as there.  A row index past the end of x raises
ValueError("gather_rows_gpu row index") before the launch (the reference
does not check).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Sequence, Union

import numpy as np
import torch

from . import capi
from .moe import _call, _ptr, _stream

VOCAB_SIZE = 32064                 # reference include/config.h:7
MAX_POSITION_EMBEDDINGS = 4096     # reference include/config.h:16


@dataclass
class PrefixPlan:
    """The trie walk's outputs (reference src/model.cu:79-117 locals)."""
    seq_lens: np.ndarray       # int64 [batch]
    offsets: np.ndarray        # int64 [batch], packed row of each sequence's first token
    token_node: np.ndarray     # uint32 [total]: node of each packed token row
    node_token: np.ndarray     # uint32 [nodes]: token id of each node
    node_depth: np.ndarray     # uint32 [nodes]: depth (RoPE position) of each node
    node_anc: Optional[np.ndarray]  # uint32 [nodes, max_len]: chain root .. node, then zeros
    max_len: int

    @property
    def nodes(self) -> int:
        return int(self.node_token.shape[0])

    @property
    def last_rows(self) -> np.ndarray:
        """Node of each sequence's last token (reference src/model.cu:148-151)."""
        return self.token_node[self.offsets + self.seq_lens - 1]


def node_parents_and_runs(plan: PrefixPlan):
    """Each node's parent (the node of the previous token of a sequence that
    contains it; 0 for depth-0 nodes) and the first node of its run of
    consecutive ids (n itself when n has depth 0 or its parent is not
    n - 1): the inputs of the device ancestor table (aps_prefix_ancestors)."""
    n = plan.nodes
    parent = np.zeros(max(n, 1), np.uint32)[:n]
    tn = plan.token_node.astype(np.int64)
    starts = np.zeros(tn.shape[0], bool)
    starts[plan.offsets] = True
    inner = np.nonzero(~starts)[0]
    parent[tn[inner]] = tn[inner - 1]
    idx = np.arange(n, dtype=np.int64)
    is_start = (plan.node_depth == 0) | (parent.astype(np.int64) != idx - 1)
    run_start = np.maximum.accumulate(np.where(is_start, idx, 0)).astype(np.uint32) if n else parent.copy()
    return parent, run_start


def ancestors_gpu(plan: PrefixPlan, device):
    """The ancestor table [nodes][max_len] (int32 view of uint32) built on
    the device from the plan's parents and runs, equal to the host table.
    It runs on torch's current stream of `device`, the stream the input
    uploads are ordered on and the one whose caching allocator takes them
    back on return."""
    parent, run_start = node_parents_and_runs(plan)
    n, stride = plan.nodes, max(plan.max_len, 1)
    to_dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(device)
    p_d, d_d, r_d = to_dev(parent), to_dev(plan.node_depth), to_dev(run_start)
    anc = torch.empty((n, stride), dtype=torch.int32, device=device)
    _call(capi.lib().aps_prefix_ancestors(_ptr(p_d), _ptr(d_d), _ptr(r_d), n, stride, _ptr(anc),
                                          _stream(anc.device)))
    return anc


def prefix_dedup(input_ids: Sequence[Sequence[int]], with_ancestors: bool = True,
                 vocab_size: int = VOCAB_SIZE, max_positions: int = MAX_POSITION_EMBEDDINGS) -> PrefixPlan:
    """The prefix trie of a prompt batch (reference src/model.cu:44-117)."""
    batch = len(input_ids)
    if batch == 0:
        raise RuntimeError("generate received an empty input batch")
    seqs = [np.asarray(s, dtype=np.int64).reshape(-1) for s in input_ids]
    seq_lens = np.array([s.shape[0] for s in seqs], dtype=np.int64)
    seq_offsets = np.zeros(batch + 1, dtype=np.int64)
    np.cumsum(seq_lens, out=seq_offsets[1:])
    total = int(seq_offsets[-1])
    flat = np.concatenate(seqs) if total else np.zeros(0, np.int64)
    # ids outside int32 cannot be in the vocabulary: clip to a value that fails the same check
    ids = np.where((flat < 0) | (flat >= vocab_size), -1, flat).astype(np.int32)
    max_len = int(seq_lens.max()) if batch else 0
    token_node = np.empty(max(total, 1), np.uint32)
    node_token = np.empty(max(total, 1), np.uint32)
    node_depth = np.empty(max(total, 1), np.uint32)
    anc_ok = with_ancestors and 0 < max_len <= max_positions
    node_anc = np.empty((max(total, 1), max(max_len, 1)), np.uint32) if anc_ok else None
    nodes = ctypes.c_int64(0)
    _call(capi.lib().aps_prefix_dedup(
        ids.ctypes.data_as(ctypes.c_void_p), seq_offsets.ctypes.data_as(ctypes.c_void_p), batch, vocab_size,
        max_positions, token_node.ctypes.data_as(ctypes.c_void_p), node_token.ctypes.data_as(ctypes.c_void_p),
        node_depth.ctypes.data_as(ctypes.c_void_p),
        node_anc.ctypes.data_as(ctypes.c_void_p) if node_anc is not None else None, max(max_len, 1),
        ctypes.byref(nodes)))
    n = nodes.value
    return PrefixPlan(seq_lens=seq_lens, offsets=seq_offsets[:-1].copy(), token_node=token_node[:total],
                      node_token=node_token[:n].copy(), node_depth=node_depth[:n].copy(),
                      node_anc=node_anc[:n].copy() if node_anc is not None else None, max_len=max_len)


class RowIndexBuffer:
    """A row-index map uploaded to the device once and reused by many
    gathers (reference include/tensor.h:119-137)."""

    def __init__(self, rows: Union[Sequence[int], np.ndarray], device: Union[str, torch.device] = "cuda"):
        r = np.asarray(rows, dtype=np.int64).reshape(-1)
        if r.size and (r.min() < 0 or r.max() > 0xFFFFFFFF):
            raise ValueError("gather_rows_gpu row index")
        self.size = int(r.size)
        self.max_row = int(r.max()) if r.size else -1
        self.data = torch.from_numpy(r.astype(np.uint32).view(np.int32)).to(device)

    def empty(self) -> bool:
        return self.size == 0


def gather_rows_gpu(x: torch.Tensor, rows: Union[RowIndexBuffer, Sequence[int], np.ndarray],
                    out: torch.Tensor) -> torch.Tensor:
    """out[i] = x[rows[i]] over the last dimension (reference
    src/tensor.cu:3379-3386 for a host index list, 3420-3426 for a
    RowIndexBuffer).  fp32, contiguous; out holds len(rows) rows."""
    if not isinstance(rows, RowIndexBuffer):
        rows = RowIndexBuffer(rows, x.device)
    if rows.empty():
        return out
    if x.dtype != torch.float32 or out.dtype != torch.float32 or not x.is_contiguous() or not out.is_contiguous():
        raise ValueError("gather_rows_gpu expects contiguous fp32 tensors")
    h = x.shape[-1]
    x_rows = x.numel() // h if h else 0
    if out.numel() != rows.size * h:
        raise ValueError("gather_rows_gpu output size")
    if rows.max_row >= x_rows:
        raise ValueError("gather_rows_gpu row index")
    _call(capi.lib().aps_gather_rows(_ptr(x), x_rows, h, _ptr(rows.data), rows.size, _ptr(out), _stream(x.device)))
    return out
