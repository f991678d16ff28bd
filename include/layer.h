// Linear, PhiMLP, PhiMoE, PhiAttention and PhiDecoderLayer over the C ABI
// (reference include/layer.h:11-95).
//
// The forward signatures are the reference's, and so are the ModelLoader
// constructors (src/layer.cu:44-47, 94-111: the same tensor names); the
// constructors that take the weight tensors directly serve callers without
// a model.bin.  forward(..., use_gpu = true) runs the
// HIP path; the reference's CPU branch (use_gpu = false) is not provided and
// throws std::invalid_argument.
#pragma once

#include <cstddef>
#include <vector>

#include <string>

#include "config.h"
#include "model_loader.h"
#include "tensor.h"

// A dense layer y = x W^T (+ b) (reference include/layer.h:11-21,
// src/layer.cu:13-42).  The GPU path is one fp32 FMA chain per output over k
// ascending with the bias added once, the reference GPU kernel's arithmetic.
// The loader constructor loads the bias only when the file holds it, as the
// reference does (a bias-less lm_head is valid).
class Linear {
public:
    Linear() = default;
    Linear(Tensor weight, Tensor bias = Tensor());
    Linear(const ModelLoader& loader, const std::string& weight, const std::string& bias = "");
    void forward(const Tensor& x, Tensor& y, bool use_gpu = false) const;
    const Tensor& weight() const { return weight_; }
    const Tensor& bias() const { return bias_; }

private:
    Tensor weight_;
    Tensor bias_;
};

class PhiMLP {
public:
    // w1, w3: [F][H]; w2: [H][F] (nn.Linear layout).
    PhiMLP(Tensor w1, Tensor w2, Tensor w3);
    // <prefix>.w1.weight, <prefix>.w2.weight, <prefix>.w3.weight
    PhiMLP(const ModelLoader& loader, const std::string& prefix);
    // y = w2 . (silu(w1 . x) * (w3 . x)) row by row; y takes x's shape.  The
    // GPU path keeps the reference's fp32 arithmetic (src/layer.cu:49-67 with
    // matmul_pair_silu_gpu), so it matches the reference bit for bit.
    void forward(const Tensor& x, Tensor& y, bool use_gpu = false) const;
    const Tensor& w1() const { return w1_; }
    const Tensor& w2() const { return w2_; }
    const Tensor& w3() const { return w3_; }

private:
    Tensor w1_, w2_, w3_;
    mutable std::size_t dense_handle_ = 0;  // one-expert weight set, registered on first GPU use
};

class PhiMoE {
public:
    // gate: [NUM_EXPERTS][H]; experts: NUM_EXPERTS PhiMLPs.  `compute` picks
    // the expert FFN kernels: APS_DTYPE_F32 (the reference's arithmetic) or
    // APS_DTYPE_BF16 (MFMA, fp32 accumulate).  Routing is exact either way.
    PhiMoE(Tensor gate, std::vector<PhiMLP> experts, aps_dtype compute = APS_DTYPE_F32);
    // model.layers.<layer_idx>.block_sparse_moe.gate.weight and
    // ....experts.<e>.{w1,w2,w3}.weight for e < NUM_EXPERTS
    PhiMoE(const ModelLoader& loader, std::size_t layer_idx, aps_dtype compute = APS_DTYPE_F32);
    // y [rows][H] = sum over the two routed experts of 0.5 * expert(x): the
    // reference's router GEMM and grouped block (src/layer.cu:113-121) as one
    // fused call (aps_moe_forward: the router kernel also routes, and for
    // bf16 compute writes the FFN's bf16 copy of x), with the same logits,
    // routes and, for fp32 compute, the same output bits.
    void forward(const Tensor& x, Tensor& y, bool use_gpu = false) const;

private:
    Tensor gate_;
    std::vector<PhiMLP> experts_;
    std::size_t gpu_weights_handle_ = 0;
};

// The prefix trie's device arrays for attention on trie-node rows
// (reference include/layer.h:57-63).
struct PrefixExpansion {
    const tensor_ops::RowIndexBuffer* node_pos = nullptr;  // node row -> depth
    const tensor_ops::RowIndexBuffer* node_anc = nullptr;  // node row -> chain
    std::size_t anc_stride = 0;
    std::size_t max_seq = 0;
    bool active() const { return node_anc != nullptr; }
};

// Self-attention of the decoder layer (reference include/layer.h:65-75,
// src/layer.cu:150-264): q/k/v/o projections with bias, RoPE and GQA-4
// attention.  With an active expansion the rows are prefix-trie nodes (RoPE
// at node depths, attention over ancestor chains: the reference's prefill);
// without one they are the sequences of seq_lens packed one after another
// (positions restart per sequence, keys never cross a sequence).  The
// expansion's positions must be < max_seq and < anc_stride and its
// ancestors < the row count (std::invalid_argument("PhiAttention prefix
// expansion") otherwise).
class PhiAttention {
public:
    PhiAttention(const ModelLoader& loader, std::size_t layer_idx);
    PhiAttention(Linear q_proj, Linear k_proj, Linear v_proj, Linear o_proj);
    void forward(const Tensor& x, Tensor& y, const std::vector<std::size_t>& seq_lens, bool use_gpu = false,
                 const PrefixExpansion& expansion = {}) const;

private:
    Linear q_proj_, k_proj_, v_proj_, o_proj_;
};

// One decoder layer (reference include/layer.h:77-95, src/layer.cu:266-326):
// LayerNorm -> attention -> residual add + LayerNorm -> MoE.  Norms are
// LayerNorm with bias, eps NORM_EPS.
class PhiDecoderLayer {
public:
    // model.layers.<i>.{input_layernorm,post_attention_layernorm}.{weight,bias},
    // the layer's attention and MoE block; moe_compute as in PhiMoE.
    PhiDecoderLayer(const ModelLoader& loader, std::size_t layer_idx, aps_dtype moe_compute = APS_DTYPE_F32);
    PhiDecoderLayer(Tensor input_norm_weight, Tensor input_norm_bias, Tensor post_norm_weight, Tensor post_norm_bias,
                    PhiAttention attention, PhiMoE moe);
    // Residual-carrying form of the packed GPU prefill: on entry the layer
    // input is x (has_carry false) or x + carry (has_carry true, the add
    // folded into the input LayerNorm); on exit x holds the MoE output and
    // carry the attention residual (attention output + layer input), whose
    // add rides into the next LayerNorm.
    void forward_carry(Tensor& x, Tensor& carry, bool has_carry, const std::vector<std::size_t>& seq_lens,
                       const PrefixExpansion& expansion) const;
    // y = MoE(LN(attn + x)) + (attn + x), attn = attention(LN(x)).  GPU only
    // (use_gpu = false throws std::invalid_argument).
    void forward(const Tensor& x, Tensor& y, const std::vector<std::size_t>& seq_lens, bool use_gpu = false,
                 const PrefixExpansion& expansion = {}) const;

private:
    Tensor input_norm_weight_, input_norm_bias_;
    Tensor post_norm_weight_, post_norm_bias_;
    PhiAttention attention_;
    PhiMoE moe_;
};
