"""Oracle of the decoder layer and of the whole model, composed from the
pinned oracle functions (test infrastructure only).

Follows the reference's order of operations:
  PhiDecoderLayer::forward_carry   src/layer.cu:273-300
  PhiDecoderLayer::forward         src/layer.cu:302-326
  PhiAttention::forward            src/layer.cu:156-264 (trie and packed paths)
  PhiTinyMoEModel::generate        src/model.cu:45-159
  PhiTinyMoEModel::forward         src/model.cu:20-37
Weights are a dict keyed by the reference's model.bin tensor names.  `moe`
computes a MoE block from (x, gate, w1, w3, w2) -- the fp32 oracle by
default; the bf16 tests pass a function that applies the bf16 rounding of
the compute path before the oracle.
"""
import numpy as np

import oracle

EPS = 1e-5
QH, KVH, HD = 16, 4, 128


def fp32_moe(x, gate, w1, w3, w2):
    return oracle.reference_path(x, gate, w1, w3, w2)["out"]


def layer_weights(W, i):
    p = f"model.layers.{i}."
    moe = p + "block_sparse_moe."
    E = W[moe + "gate.weight"].shape[0]
    return dict(
        in_w=W[p + "input_layernorm.weight"], in_b=W[p + "input_layernorm.bias"],
        post_w=W[p + "post_attention_layernorm.weight"], post_b=W[p + "post_attention_layernorm.bias"],
        attn={nm: (W[p + f"self_attn.{nm}.weight"], W[p + f"self_attn.{nm}.bias"])
              for nm in ("q_proj", "k_proj", "v_proj", "o_proj")},
        gate=W[moe + "gate.weight"],
        w1=np.stack([W[moe + f"experts.{e}.w1.weight"] for e in range(E)]),
        w2=np.stack([W[moe + f"experts.{e}.w2.weight"] for e in range(E)]),
        w3=np.stack([W[moe + f"experts.{e}.w3.weight"] for e in range(E)]),
    )


def chain_table(row_pos, anc_lists):
    """Ancestor table [rows][stride] (stride = longest chain) from the chains."""
    stride = max(len(c) for c in anc_lists)
    anc = np.zeros((len(anc_lists), stride), np.uint32)
    for r, c in enumerate(anc_lists):
        anc[r, :len(c)] = c
    return np.asarray(row_pos, np.uint32), anc, stride


def packed_chains(seq_lens):
    """Positions and key chains of packed sequences: row r of a sequence
    starting at o sits at position p and attends to rows o .. o + p."""
    pos, chains, o = [], [], 0
    for n in seq_lens:
        for p in range(n):
            pos.append(p)
            chains.append(list(range(o, o + p + 1)))
        o += n
    return pos, chains


def attention(x, L, row_pos, anc, stride):
    q = oracle.linear(x, *L["attn"]["q_proj"])
    k = oracle.linear(x, *L["attn"]["k_proj"])
    v = oracle.linear(x, *L["attn"]["v_proj"])
    c, s = oracle.rope_table(stride, HD)
    q = oracle.rope_tree(q, row_pos, QH, HD, c, s)
    k = oracle.rope_tree(k, row_pos, KVH, HD, c, s)
    att = oracle.attention_tree(q, k, v, row_pos, anc, stride, QH, KVH, HD)
    return oracle.linear(att, *L["attn"]["o_proj"])


def layer_carry(x, carry, L, row_pos, anc, stride, moe=fp32_moe):
    """forward_carry: returns (new x = MoE output, new carry = attn + input)."""
    if carry is None:
        normed, v, _, _ = oracle.layer_norm(x, L["in_w"], L["in_b"], EPS)
    else:
        normed, v, _, _ = oracle.layer_norm(x, L["in_w"], L["in_b"], EPS, residual=carry)
    attn = attention(normed, L, row_pos, anc, stride)
    post, attn_res, _, _ = oracle.layer_norm(attn, L["post_w"], L["post_b"], EPS, residual=v)
    return moe(post, L["gate"], L["w1"], L["w3"], L["w2"]), attn_res


def generate(W, prompts, n_layers, moe=fp32_moe):
    token_node, node_token, node_depth, node_anc = oracle.prefix_dedup(prompts)
    row_pos, anc, stride = chain_table(node_depth, node_anc)
    h = oracle.gather_rows(W["model.embed_tokens.weight"], node_token)
    carry = None
    for i in range(n_layers):
        h, carry = layer_carry(h, carry, layer_weights(W, i), row_pos, anc, stride, moe)
    if carry is None:
        normed, _, _, _ = oracle.layer_norm(h, W["model.norm.weight"], W["model.norm.bias"], EPS)
    else:
        normed, _, _, _ = oracle.layer_norm(h, W["model.norm.weight"], W["model.norm.bias"], EPS, residual=carry)
    offs = np.cumsum([0] + [len(p) for p in prompts])
    last = oracle.gather_rows(normed, [token_node[offs[b] + len(prompts[b]) - 1] for b in range(len(prompts))])
    return oracle.linear(last, W["lm_head.weight"], W.get("lm_head.bias"))


def forward(W, ids, n_layers, moe=fp32_moe):
    """One sequence through the packed path; layer outputs MoE + residual."""
    pos, chains = packed_chains([len(ids)])
    row_pos, anc, stride = chain_table(pos, chains)
    h = oracle.gather_rows(W["model.embed_tokens.weight"], ids)
    for i in range(n_layers):
        ff, attn_res = layer_carry(h, None, layer_weights(W, i), row_pos, anc, stride, moe)
        h = (ff + attn_res).astype(np.float32)  # one fp32 add per element
    normed, _, _, _ = oracle.layer_norm(h, W["model.norm.weight"], W["model.norm.bias"], EPS)
    return oracle.linear(normed[-1:], W["lm_head.weight"], W.get("lm_head.bias"))
