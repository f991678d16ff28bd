// The layer classes over the C ABI (declared in include/layer.h).
//
// Reference: PhiMLP::PhiMLP and forward (src/layer.cu:44-67), PhiMoE::PhiMoE
// (src/layer.cu:94-111, the tensor names) and PhiMoE::forward
// (src/layer.cu:113-121, the GPU branch), Linear (:13-42), PhiAttention
// (:150-264) and PhiDecoderLayer (:266-326).
#include "../../include/layer.h"

#include <stdexcept>
#include <string>
#include <utility>

namespace aps_cpp_detail {
void mlp_forward_gpu(std::size_t handle, const Tensor& x, std::size_t rows, Tensor& out);
std::size_t register_dense(const Tensor& w1, const Tensor& w2, const Tensor& w3);
void moe_forward_fused(std::size_t handle, const Tensor& x, const Tensor& gate, Tensor& out);
}  // namespace aps_cpp_detail

PhiMLP::PhiMLP(Tensor w1, Tensor w2, Tensor w3) : w1_(std::move(w1)), w2_(std::move(w2)), w3_(std::move(w3)) {
    if (w1_.ndim() != 2 || w3_.shape() != w1_.shape() || w2_.ndim() != 2 || w2_.size(0) != w1_.size(1) ||
        w2_.size(1) != w1_.size(0))
        throw std::invalid_argument("PhiMLP weight shapes");
}

PhiMLP::PhiMLP(const ModelLoader& loader, const std::string& prefix)
    : PhiMLP(loader.load(prefix + ".w1.weight"), loader.load(prefix + ".w2.weight"),
             loader.load(prefix + ".w3.weight")) {}

void PhiMLP::forward(const Tensor& x, Tensor& y, bool use_gpu) const {
    if (!use_gpu) throw std::invalid_argument("PhiMLP::forward: the CPU path (use_gpu = false) is not provided");
    const std::size_t h = x.size(x.ndim() - 1);
    if (h != w1_.size(1)) throw std::invalid_argument("PhiMLP::forward shape");
    const std::size_t rows = x.size() / h;
    if (!dense_handle_) dense_handle_ = aps_cpp_detail::register_dense(w1_, w2_, w3_);
    Tensor out({rows, w2_.size(0)});
    if (rows) aps_cpp_detail::mlp_forward_gpu(dense_handle_, x, rows, out);
    out.reshape(x.shape());
    y = std::move(out);
}

PhiMoE::PhiMoE(Tensor gate, std::vector<PhiMLP> experts, aps_dtype compute)
    : gate_(std::move(gate)), experts_(std::move(experts)) {
    std::vector<const Tensor*> w1, w2, w3;
    for (const PhiMLP& e : experts_) {
        w1.push_back(&e.w1());
        w2.push_back(&e.w2());
        w3.push_back(&e.w3());
    }
    gpu_weights_handle_ = tensor_ops::register_moe_weights_gpu(w1, w2, w3, compute);
}

namespace {
std::vector<PhiMLP> load_experts(const ModelLoader& loader, const std::string& base) {
    std::vector<PhiMLP> experts;
    experts.reserve(apss26::NUM_EXPERTS);
    for (std::size_t e = 0; e < apss26::NUM_EXPERTS; ++e)
        experts.emplace_back(loader, base + ".experts." + std::to_string(e));
    return experts;
}
std::string moe_base(std::size_t layer_idx) {
    return "model.layers." + std::to_string(layer_idx) + ".block_sparse_moe";
}
}  // namespace

PhiMoE::PhiMoE(const ModelLoader& loader, std::size_t layer_idx, aps_dtype compute)
    : PhiMoE(loader.load(moe_base(layer_idx) + ".gate.weight"), load_experts(loader, moe_base(layer_idx)), compute) {}

void PhiMoE::forward(const Tensor& x, Tensor& y, bool use_gpu) const {
    if (!use_gpu) throw std::invalid_argument("PhiMoE::forward: the CPU path (use_gpu = false) is not provided");
    aps_cpp_detail::moe_forward_fused(gpu_weights_handle_, x, gate_, y);
}

// ---- Linear and PhiAttention (reference src/layer.cu:21-42, 150-188) --------

Linear::Linear(Tensor weight, Tensor bias) : weight_(std::move(weight)), bias_(std::move(bias)) {
    if (weight_.ndim() != 2 || (bias_.size() && bias_.size() != weight_.size(0)))
        throw std::invalid_argument("Linear weight shapes");
}

Linear::Linear(const ModelLoader& loader, const std::string& weight, const std::string& bias)
    : Linear(loader.load(weight), !bias.empty() && loader.has(bias) ? loader.load(bias) : Tensor()) {
#ifdef USE_TC
    // built with USE_TC (USE_TC_ALL): the split-bf16 Linear for the LM head
    // and the last layer's (every layer's) attention projections, the
    // reference's selection (src/layer.cu:16-27)
#ifdef USE_TC_ALL
    const bool terminal_tc = weight == "lm_head.weight" ||
                             (weight.find("model.layers.") == 0 && weight.find(".self_attn.") != std::string::npos);
#else
    const bool terminal_tc = weight == "lm_head.weight" || weight.find("model.layers.31.self_attn.") == 0;
#endif
    if (terminal_tc) weight_.prepare_cuda_bf16_weight(true);
#endif
}

void Linear::forward(const Tensor& x, Tensor& y, bool use_gpu) const {
    if (!use_gpu) throw std::invalid_argument("Linear::forward: the CPU path (use_gpu = false) is not provided");
    const std::size_t rows = x.size() / x.size(x.ndim() - 1);
    y = Tensor({rows, weight_.size(0)});
    if (bias_.size())
        tensor_ops::matmul_transposed_bias_gpu(x, weight_, bias_, y);
    else
        tensor_ops::matmul_transposed_gpu(x, weight_, y);
}

namespace {
std::string attn_name(std::size_t layer, const char* proj, const char* what) {
    return "model.layers." + std::to_string(layer) + ".self_attn." + proj + "." + what;
}
}  // namespace

PhiAttention::PhiAttention(const ModelLoader& loader, std::size_t layer_idx)
    : q_proj_(loader, attn_name(layer_idx, "q_proj", "weight"), attn_name(layer_idx, "q_proj", "bias")),
      k_proj_(loader, attn_name(layer_idx, "k_proj", "weight"), attn_name(layer_idx, "k_proj", "bias")),
      v_proj_(loader, attn_name(layer_idx, "v_proj", "weight"), attn_name(layer_idx, "v_proj", "bias")),
      o_proj_(loader, attn_name(layer_idx, "o_proj", "weight"), attn_name(layer_idx, "o_proj", "bias")) {}

PhiAttention::PhiAttention(Linear q_proj, Linear k_proj, Linear v_proj, Linear o_proj)
    : q_proj_(std::move(q_proj)), k_proj_(std::move(k_proj)), v_proj_(std::move(v_proj)), o_proj_(std::move(o_proj)) {}

void PhiAttention::forward(const Tensor& x, Tensor& y, const std::vector<std::size_t>& seq_lens, bool use_gpu,
                           const PrefixExpansion& expansion) const {
    if (!use_gpu) throw std::invalid_argument("PhiAttention::forward: the CPU path (use_gpu = false) is not provided");
    const std::size_t s = x.size(0);
    if (expansion.active()) {
        // the kernels clamp out-of-range device indices for memory safety
        // only; the expansion's extremes are known on the host, so check them
        if (!expansion.node_pos || expansion.node_pos->size() != s || expansion.node_anc->size() < s * expansion.anc_stride ||
            expansion.anc_stride == 0 || expansion.node_pos->max_row() >= expansion.max_seq ||
            expansion.node_pos->max_row() >= expansion.anc_stride || expansion.node_anc->max_row() >= s)
            throw std::invalid_argument("PhiAttention prefix expansion");
    }
    Tensor q, k, v;
    q_proj_.forward(x, q, true);
    // k and v as one pair when neither carries the bf16 copy (reference
    // src/layer.cu:161-172); the pair needs both biases
    const std::size_t nk = k_proj_.weight().size(0), nv = v_proj_.weight().size(0);
    const bool fuse_kv = !k_proj_.weight().has_cuda_bf16_weight() && !v_proj_.weight().has_cuda_bf16_weight() &&
                         nk == nv && k_proj_.bias().size() == nk && v_proj_.bias().size() == nv;
    if (fuse_kv) {
        k = Tensor({s, nk});
        v = Tensor({s, nv});
        tensor_ops::matmul_pair_bias_gpu(x, k_proj_.weight(), k_proj_.bias(), k, v_proj_.weight(), v_proj_.bias(), v);
    } else {
        k_proj_.forward(x, k, true);
        v_proj_.forward(x, v, true);
    }
    Tensor out({s, apss26::NUM_ATTENTION_HEADS * apss26::HEAD_DIM});
    if (expansion.active()) {
        // rows are trie nodes: RoPE at the node depth, keys along the chain
        tensor_ops::apply_rope_tree_gpu(q, k, expansion.node_pos->data(), s, expansion.max_seq,
                                        apss26::NUM_ATTENTION_HEADS, apss26::NUM_KV_HEADS, apss26::HEAD_DIM,
                                        apss26::ROPE_THETA);
        tensor_ops::attention_tree_gpu(q, k, v, out, expansion.node_pos->data(), expansion.node_anc->data(),
                                       expansion.anc_stride, s, expansion.max_seq, apss26::NUM_ATTENTION_HEADS,
                                       apss26::NUM_KV_HEADS, apss26::HEAD_DIM);
    } else {
        // rows are the packed sequences of seq_lens
        tensor_ops::apply_rope_gpu(q, k, seq_lens, apss26::NUM_ATTENTION_HEADS, apss26::NUM_KV_HEADS,
                                   apss26::HEAD_DIM, apss26::ROPE_THETA);
        tensor_ops::attention_gpu(q, k, v, out, seq_lens, apss26::NUM_ATTENTION_HEADS, apss26::NUM_KV_HEADS,
                                  apss26::HEAD_DIM);
    }
    o_proj_.forward(out, y, true);
}

// ---- PhiDecoderLayer (reference src/layer.cu:266-326) -----------------------

namespace {
std::string layer_name(std::size_t layer, const char* what) {
    return "model.layers." + std::to_string(layer) + "." + what;
}
}  // namespace

PhiDecoderLayer::PhiDecoderLayer(const ModelLoader& loader, std::size_t layer_idx, aps_dtype moe_compute)
    : PhiDecoderLayer(loader.load(layer_name(layer_idx, "input_layernorm.weight")),
                      loader.load(layer_name(layer_idx, "input_layernorm.bias")),
                      loader.load(layer_name(layer_idx, "post_attention_layernorm.weight")),
                      loader.load(layer_name(layer_idx, "post_attention_layernorm.bias")),
                      PhiAttention(loader, layer_idx), PhiMoE(loader, layer_idx, moe_compute)) {}

PhiDecoderLayer::PhiDecoderLayer(Tensor input_norm_weight, Tensor input_norm_bias, Tensor post_norm_weight,
                                 Tensor post_norm_bias, PhiAttention attention, PhiMoE moe)
    : input_norm_weight_(std::move(input_norm_weight)),
      input_norm_bias_(std::move(input_norm_bias)),
      post_norm_weight_(std::move(post_norm_weight)),
      post_norm_bias_(std::move(post_norm_bias)),
      attention_(std::move(attention)),
      moe_(std::move(moe)) {}

void PhiDecoderLayer::forward_carry(Tensor& x, Tensor& carry, bool has_carry,
                                    const std::vector<std::size_t>& seq_lens,
                                    const PrefixExpansion& expansion) const {
    // layer input: x, or x + carry folded into the input norm (x += carry in place)
    Tensor normed(x.shape());
    if (has_carry)
        tensor_ops::add_layer_norm_gpu(x, carry, input_norm_weight_, input_norm_bias_, apss26::NORM_EPS, normed);
    else
        tensor_ops::layer_norm_gpu(x, input_norm_weight_, input_norm_bias_, apss26::NORM_EPS, normed);
    Tensor attn;
    attention_.forward(normed, attn, seq_lens, true, expansion);
    // attn += layer input; the post-attention norm of that feeds the MoE
    Tensor post(attn.shape());
    tensor_ops::add_layer_norm_gpu(attn, x, post_norm_weight_, post_norm_bias_, apss26::NORM_EPS, post);
    Tensor ff;
    moe_.forward(post, ff, true);
    x = std::move(ff);
    carry = std::move(attn);
}

void PhiDecoderLayer::forward(const Tensor& x, Tensor& y, const std::vector<std::size_t>& seq_lens, bool use_gpu,
                              const PrefixExpansion& expansion) const {
    if (!use_gpu)
        throw std::invalid_argument("PhiDecoderLayer::forward: the CPU path (use_gpu = false) is not provided");
    Tensor h = x, carry;
    forward_carry(h, carry, false, seq_lens, expansion);
    tensor_ops::add_inplace_gpu(h, carry);  // MoE output + residual
    y = std::move(h);
}
