// PhiMLP and PhiMoE layers over the C ABI (reference include/layer.h:23-43).
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
// src/layer.cu:21-42).  The GPU path is one fp32 FMA chain per output over k
// ascending with the bias added once, the reference GPU kernel's arithmetic.
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
    // y [rows][H] = sum over the two routed experts of 0.5 * expert(x).
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
// src/layer.cu:150-188): q/k/v/o projections with bias, RoPE and GQA
// attention.  This build provides the prefix-trie path (expansion.active():
// RoPE at node depths, attention over ancestor chains, as the reference's
// prefill); without an expansion forward throws std::invalid_argument.
class PhiAttention {
public:
    PhiAttention(const ModelLoader& loader, std::size_t layer_idx);
    PhiAttention(Linear q_proj, Linear k_proj, Linear v_proj, Linear o_proj);
    void forward(const Tensor& x, Tensor& y, const std::vector<std::size_t>& seq_lens, bool use_gpu = false,
                 const PrefixExpansion& expansion = {}) const;

private:
    Linear q_proj_, k_proj_, v_proj_, o_proj_;
};
