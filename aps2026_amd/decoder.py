"""Decoder layer and whole-model prefill over the C ABI: the Python mirror of
include/layer.h's PhiDecoderLayer and include/model.h's PhiTinyMoEModel.

Reference order of operations (file:line in the reference tree):
  PhiDecoderLayer::forward_carry   src/layer.cu:273-300
  PhiAttention::forward (trie)     src/layer.cu:156-194
  PhiTinyMoEModel::generate        src/model.cu:45-159

A prefill runs on the rows of the prompts' prefix trie (one row per
distinct prefix, aps2026_amd.prefix): gather the embedding rows of the
nodes, then per layer
    normed = LN(x)            (first layer)   or  LN(x += carry)
    q, k, v = normed W^T + b  (fp32 FMA chains, the reference's arithmetic)
    RoPE(q, k) at node depths; attention over ancestor chains (GQA-4)
    attn = att W_o^T + b_o
    post = LN(attn += x)      (attn becomes the carried residual)
    x = MoE(post)             (router, top-2, dispatch, experts, combine)
then the final LN of x + carry, each prompt's last row and the LM head.
Every buffer is allocated once per row count (Buffers) and every step is a
sequence of C-ABI launches on one stream with no host synchronisation, so a
prefill can be timed or captured as it is.  Activations are fp32; the MoE
experts compute in the weight set's dtype (fp32, or bf16 with the router
reading fp32 x exactly and the experts a bf16 copy of it).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import capi, prefix
from .attention import HEAD_DIM, NUM_ATTENTION_HEADS, NUM_KV_HEADS, ROPE_THETA, SLIDING_WINDOW, _device_table
from .moe import NORM_EPS, MoeWeights, _call, register_moe_weights_gpu

QD = NUM_ATTENTION_HEADS * HEAD_DIM   # 2048: q and attention-output width
KD = NUM_KV_HEADS * HEAD_DIM          # 512: k and v width


def _p(t: Optional[torch.Tensor]) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


@dataclass
class LayerWeights:
    """One decoder layer's weights on the device (fp32 except the registered
    expert set), under the reference's model.bin names."""
    in_w: torch.Tensor
    in_b: torch.Tensor
    post_w: torch.Tensor
    post_b: torch.Tensor
    proj: Dict[str, Tuple[torch.Tensor, torch.Tensor]]   # q_proj, k_proj, v_proj, o_proj: (weight, bias)
    gate: torch.Tensor
    moe: MoeWeights

    def release(self) -> None:
        self.moe.release()


def layer_from_tensors(W: Dict[str, torch.Tensor], i: int, moe_dtype=torch.float32) -> LayerWeights:
    """model.layers.<i>.* of a name -> tensor dict (device or host fp32)."""
    dev = W["model.layers.%d.self_attn.q_proj.weight" % i].device
    p = f"model.layers.{i}."
    m = p + "block_sparse_moe."
    f32 = lambda t: t.to(device=dev, dtype=torch.float32).contiguous()
    E = W[m + "gate.weight"].shape[0]
    experts = [[f32(W[m + f"experts.{e}.{nm}.weight"]) for e in range(E)] for nm in ("w1", "w2", "w3")]
    moe = register_moe_weights_gpu(*experts, compute_dtype=moe_dtype)
    del experts
    return LayerWeights(
        in_w=f32(W[p + "input_layernorm.weight"]), in_b=f32(W[p + "input_layernorm.bias"]),
        post_w=f32(W[p + "post_attention_layernorm.weight"]), post_b=f32(W[p + "post_attention_layernorm.bias"]),
        proj={nm: (f32(W[p + f"self_attn.{nm}.weight"]), f32(W[p + f"self_attn.{nm}.bias"]))
              for nm in ("q_proj", "k_proj", "v_proj", "o_proj")},
        gate=f32(W[m + "gate.weight"]), moe=moe)


def random_layer(H: int, F: int, E: int, device, generator: torch.Generator, moe_dtype=torch.bfloat16,
                 std: float = 0.02) -> LayerWeights:
    """A random-init layer drawn on the device: linear and expert weights and
    the projection biases ~N(0, std), LayerNorm weight 1 and bias 0 (the
    usual initialisation).  The fp32 expert weights are freed once the
    packed set is registered."""
    rn = lambda *shape: (std * torch.randn(shape, generator=generator, device=device)).contiguous()
    proj = {nm: (rn(o, k), rn(o)) for nm, (o, k) in
            (("q_proj", (QD, H)), ("k_proj", (KD, H)), ("v_proj", (KD, H)), ("o_proj", (H, QD)))}
    gate = rn(E, H)
    w1 = [rn(F, H) for _ in range(E)]
    w2 = [rn(H, F) for _ in range(E)]
    w3 = [rn(F, H) for _ in range(E)]
    moe = register_moe_weights_gpu(w1, w2, w3, compute_dtype=moe_dtype)
    del w1, w2, w3
    one = torch.ones(H, device=device)
    zero = torch.zeros(H, device=device)
    return LayerWeights(in_w=one, in_b=zero, post_w=one.clone(), post_b=zero.clone(), proj=proj, gate=gate, moe=moe)


@dataclass
class RowPlan:
    """Device arrays of a prefix-trie plan for attention on node rows,
    checked once on the host: positions below the ancestor stride,
    ancestors below the row count."""
    rows: int
    max_len: int
    pos: torch.Tensor        # int32 view of u32 [rows]
    anc: torch.Tensor        # int32 view of u32 [rows][max_len]
    node_token: torch.Tensor
    last_rows: torch.Tensor  # int32 view of u32 [batch]: each prompt's last node
    prompt_tokens: int

    @staticmethod
    def from_prompts(prompts: Sequence[Sequence[int]], device) -> "RowPlan":
        # the trie on the host, its ancestor table on the device (the host
        # table is nodes x max_len words: 42 MB at C4, which took longer to
        # fill, copy and upload than a layer of the model)
        plan = prefix.prefix_dedup(prompts, with_ancestors=False)
        depth = np.asarray(plan.node_depth, np.uint32)
        if depth.size and int(depth.max()) >= plan.max_len:
            raise ValueError("prefix plan out of range")
        to_dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(device)
        anc = prefix.ancestors_gpu(plan, device)
        return RowPlan(rows=plan.nodes, max_len=plan.max_len, pos=to_dev(depth), anc=anc,
                       node_token=to_dev(np.asarray(plan.node_token, np.uint32)),
                       last_rows=to_dev(np.asarray(plan.last_rows, np.uint32)),
                       prompt_tokens=int(np.asarray(plan.token_node).shape[0]))


    @staticmethod
    def packed(prompts: Sequence[Sequence[int]], device) -> "RowPlan":
        """Every token its own row, no deduplication: row r of a prompt that
        starts at row o has position p = r - o and keys o .. r (the packed
        sequences of the reference's non-trie path, written as chains)."""
        lens = [len(p) for p in prompts]
        if not lens or min(lens) == 0:
            raise ValueError("empty input")
        rows, max_len = sum(lens), max(lens)
        pos = np.concatenate([np.arange(n, dtype=np.uint32) for n in lens])
        starts = np.repeat(np.cumsum([0] + lens[:-1]).astype(np.uint32), lens)
        cols = np.arange(max_len, dtype=np.uint32)[None, :]
        anc = np.where(cols <= pos[:, None], starts[:, None] + cols, 0).astype(np.uint32)
        to_dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(device)
        last = np.cumsum(lens).astype(np.uint32) - 1
        return RowPlan(rows=rows, max_len=max_len, pos=to_dev(pos), anc=to_dev(anc),
                       node_token=to_dev(np.concatenate([np.asarray(p, np.uint32) for p in prompts])),
                       last_rows=to_dev(last), prompt_tokens=rows)


def routes_view(b: "Buffers", moe: MoeWeights) -> torch.Tensor:
    """The routes [rows][2] (u8) the last MoE block wrote into b.ws."""
    off = moe.layout(b.rows).routes
    return b.ws[off:off + 2 * b.rows].view(b.rows, 2)


@dataclass
class Buffers:
    """Activations of one prefill at a row count, allocated once."""
    rows: int
    x: torch.Tensor          # residual stream / MoE output [rows][H]
    carry: torch.Tensor      # attention residual [rows][H]
    normed: torch.Tensor     # [rows][H]
    q: torch.Tensor          # [rows][QD]
    k: torch.Tensor          # [rows][KD]
    v: torch.Tensor
    att: torch.Tensor        # attention output [rows][QD]
    post: torch.Tensor       # MoE input [rows][H]
    ws: torch.Tensor         # MoE workspace (shared by the layers)
    xs: Optional[torch.Tensor] = None   # split-bf16 projections: x_hi, x_lo of one input

    def split(self, src: torch.Tensor, stream) -> torch.Tensor:
        """src [rows][n] fp32 -> its bf16 hi / lo split in xs (grown on demand)."""
        n = src.numel()
        if self.xs is None or self.xs.numel() < 2 * n:
            self.xs = torch.empty(2 * n, dtype=torch.int16, device=src.device)
        _call(capi.lib().aps_linear_tc_split(_p(src), self.rows, src.shape[1], _p(self.xs), stream))
        return self.xs

    @staticmethod
    def allocate(rows: int, H: int, moe: MoeWeights, device) -> "Buffers":
        e = lambda *s: torch.empty(s, dtype=torch.float32, device=device)
        ws = torch.empty(max(moe.layout(rows).total_bytes, 1), dtype=torch.uint8, device=device)
        return Buffers(rows, e(rows, H), e(rows, H), e(rows, H), e(rows, QD), e(rows, KD), e(rows, KD),
                       e(rows, QD), e(rows, H), ws)


class DecoderLayer:
    """PhiDecoderLayer over the C ABI (reference include/layer.h:77-95).

    tc_terms: None for the fp32 projections (the reference's default build);
    3 or 4 for the split-bf16 Linear on the q/k/v/o projections (the
    reference's USE_TC / USE_TC_ALL tensor-core path, src/layer.cu:16-27,
    src/tensor.cu:514-584), whose weights are packed here once."""

    def __init__(self, w: LayerWeights, tc_terms: Optional[int] = None):
        self.w = w
        self.H = w.in_w.numel()
        self.tc_terms = tc_terms
        self.tc = {}
        if tc_terms is not None:
            from .attention import linear_tc_prepare
            self.tc = {nm: linear_tc_prepare(wt) for nm, (wt, _) in w.proj.items()}

    def _project(self, b: Buffers, src: torch.Tensor, names, stream) -> None:
        """The projections of one input: fp32 chains, or the split products
        (x split once for all of them)."""
        L, T, K = capi.lib(), b.rows, src.shape[1]
        if self.tc:
            # every output of the input in one launch (their column blocks share the grid)
            xs = b.split(src, stream)
            cnt = len(names)
            vp = ctypes.c_void_p * cnt
            _call(L.aps_linear_tc_multi(_p(xs), T, K, cnt, vp(*[_p(self.tc[nm]) for nm, _, _ in names]),
                                        vp(*[_p(self.w.proj[nm][1]) for nm, _, _ in names]),
                                        (ctypes.c_int32 * cnt)(*[n for _, _, n in names]), int(self.tc_terms == 4),
                                        vp(*[_p(dst) for _, dst, _ in names]), stream))
        else:
            # an output wide enough to fill the grid alone (q, o) by itself;
            # the narrow ones (k and v) share one grid, so that no CU holds a
            # third workgroup of one while others hold two
            wide = [x for x in names if x[2] >= 2048]
            narrow = [x for x in names if x[2] < 2048]
            for nm, dst, n in wide:
                _call(L.aps_linear(_p(src), _p(self.w.proj[nm][0]), _p(self.w.proj[nm][1]), T, K, n, _p(dst),
                                   stream))
            if narrow:
                cnt = len(narrow)
                vp = ctypes.c_void_p * cnt
                _call(L.aps_linear_multi(_p(src), T, K, cnt, vp(*[_p(self.w.proj[nm][0]) for nm, _, _ in narrow]),
                                         vp(*[_p(self.w.proj[nm][1]) for nm, _, _ in narrow]),
                                         (ctypes.c_int32 * cnt)(*[n for _, _, n in narrow]),
                                         vp(*[_p(dst) for _, dst, _ in narrow]), stream))

    def attention(self, b: Buffers, plan: RowPlan, stream) -> None:
        """normed -> att (projections, RoPE, tree attention)."""
        L, T, H, w = capi.lib(), b.rows, self.H, self.w
        self._project(b, b.normed, (("q_proj", b.q, QD), ("k_proj", b.k, KD), ("v_proj", b.v, KD)), stream)
        c, s = _device_table(b.q.device, plan.max_len, HEAD_DIM, ROPE_THETA)
        _call(L.aps_rope_tree(_p(b.q), _p(b.k), _p(plan.pos), T, NUM_ATTENTION_HEADS, NUM_KV_HEADS, HEAD_DIM,
                              _p(c), _p(s), c.shape[0], stream))
        _call(L.aps_attention_tree(_p(b.q), _p(b.k), _p(b.v), _p(b.att), _p(plan.pos), _p(plan.anc), plan.max_len,
                                   T, NUM_ATTENTION_HEADS, NUM_KV_HEADS, HEAD_DIM, SLIDING_WINDOW, stream))

    def forward_carry(self, b: Buffers, plan: RowPlan, has_carry: bool, stream) -> None:
        """In place on b: on entry the layer input is b.x (+ b.carry when
        has_carry); on exit b.x is the MoE output and b.carry the attention
        residual."""
        L, T, H, w = capi.lib(), b.rows, self.H, self.w
        if has_carry:
            _call(L.aps_add_layer_norm(_p(b.x), _p(b.carry), _p(w.in_w), _p(w.in_b), T, H, ctypes.c_float(NORM_EPS),
                                       _p(b.normed), stream))
        else:
            _call(L.aps_layer_norm(_p(b.x), _p(w.in_w), _p(w.in_b), T, H, ctypes.c_float(NORM_EPS), _p(b.normed),
                                   stream))
        self.attention(b, plan, stream)
        # attn = att W_o^T + b_o into carry, then carry += x and post = LN(carry)
        self._project(b, b.att, (("o_proj", b.carry, H),), stream)
        _call(L.aps_add_layer_norm(_p(b.carry), _p(b.x), _p(w.post_w), _p(w.post_b), T, H, ctypes.c_float(NORM_EPS),
                                   _p(b.post), stream))
        _call(L.aps_moe_forward(w.moe.handle, _p(b.post), capi.DTYPE_F32, _p(w.gate), T, _p(b.x), capi.DTYPE_F32,
                                _p(b.ws), b.ws.numel(), stream))


class Model:
    """PhiTinyMoEModel's prefill (reference include/model.h:7-27,
    src/model.cu:45-159) over any number of layers."""

    def __init__(self, embeddings: torch.Tensor, norm_w: torch.Tensor, norm_b: torch.Tensor,
                 lm_head_w: torch.Tensor, lm_head_b: Optional[torch.Tensor], layers: List[LayerWeights],
                 tc: str = "off"):
        """tc: "off" (fp32 projections, the reference's default build), "tc"
        (the split-bf16 Linear, three products, for the LM head and layer
        31's attention projections: the reference's USE_TC) or "all" (four
        products, the LM head and every layer's attention projections:
        USE_TC_ALL)."""
        if tc not in ("off", "tc", "all"):
            raise ValueError("tc is 'off', 'tc' or 'all'")
        self.emb, self.norm_w, self.norm_b = embeddings, norm_w, norm_b
        self.head_w, self.head_b = lm_head_w, lm_head_b
        terms = None if tc == "off" else (4 if tc == "all" else 3)
        self.layers = [DecoderLayer(w, terms if (tc == "all" or (tc == "tc" and i == 31)) else None)
                       for i, w in enumerate(layers)]
        self.head_terms = terms
        self.head_tc = None
        if terms is not None:
            from .attention import linear_tc_prepare
            self.head_tc = linear_tc_prepare(lm_head_w)
        self.H = embeddings.shape[1]
        self._bufs: Dict[int, Buffers] = {}

    def buffers(self, rows: int) -> Buffers:
        b = self._bufs.get(rows)
        if b is None:
            b = Buffers.allocate(rows, self.H, self.layers[0].w.moe, self.emb.device)
            self._bufs[rows] = b
        return b

    def prefill(self, plan: RowPlan, on_layer=None) -> torch.Tensor:
        """logits [batch][vocab] of each prompt's last token; launches only
        (the outputs come from torch's caching allocator).  on_layer(i, b),
        when given, runs after layer i's launches (for example to copy its
        routes out of the shared workspace on the same stream)."""
        L, dev = capi.lib(), self.emb.device
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        b = self.buffers(plan.rows)
        T, H = plan.rows, self.H
        _call(L.aps_gather_rows(_p(self.emb), self.emb.shape[0], H, _p(plan.node_token), T, _p(b.x), stream))
        for i, layer in enumerate(self.layers):
            layer.forward_carry(b, plan, i > 0, stream)
            if on_layer is not None:
                on_layer(i, b)
        if self.layers:
            _call(L.aps_add_layer_norm(_p(b.x), _p(b.carry), _p(self.norm_w), _p(self.norm_b), T, H,
                                       ctypes.c_float(NORM_EPS), _p(b.normed), stream))
        else:
            _call(L.aps_layer_norm(_p(b.x), _p(self.norm_w), _p(self.norm_b), T, H, ctypes.c_float(NORM_EPS),
                                   _p(b.normed), stream))
        batch = plan.last_rows.shape[0]
        rows_out = torch.empty((batch, H), dtype=torch.float32, device=dev)
        _call(L.aps_gather_rows(_p(b.normed), T, H, _p(plan.last_rows), batch, _p(rows_out), stream))
        V = self.head_w.shape[0]
        logits = torch.empty((batch, V), dtype=torch.float32, device=dev)
        if self.head_tc is not None:
            xs = torch.empty(2 * batch * H, dtype=torch.int16, device=dev)
            _call(L.aps_linear_tc_split(_p(rows_out), batch, H, _p(xs), stream))
            _call(L.aps_linear_tc(_p(xs), batch, H, _p(self.head_tc), _p(self.head_b), V, int(self.head_terms == 4),
                                  _p(logits), stream))
        else:
            _call(L.aps_linear(_p(rows_out), _p(self.head_w), _p(self.head_b), batch, H, V, _p(logits), stream))
        return logits

    def generate(self, prompts: Sequence[Sequence[int]]) -> torch.Tensor:
        return self.prefill(RowPlan.from_prompts(prompts, self.emb.device))
