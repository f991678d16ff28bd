// PhiMLP / PhiMoE over the C ABI (declared in include/layer.h).
//
// Reference: PhiMLP::PhiMLP and forward (src/layer.cu:44-67), PhiMoE::PhiMoE
// (src/layer.cu:94-111, the tensor names) and PhiMoE::forward (src/layer.cu:113-121, the GPU
// branch: router GEMM, then moe_forward_grouped_gpu).
#include "../../include/layer.h"

#include <stdexcept>
#include <string>
#include <utility>

namespace aps_cpp_detail {
void mlp_forward_gpu(std::size_t handle, const Tensor& x, std::size_t rows, Tensor& out);
std::size_t register_dense(const Tensor& w1, const Tensor& w2, const Tensor& w3);
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
    const std::size_t rows = x.size(0);
    Tensor router({rows, apss26::NUM_EXPERTS});
    if (rows) tensor_ops::matmul_transposed_gpu(x, gate_, router);
    tensor_ops::moe_forward_grouped_gpu(x, router, gpu_weights_handle_, y);
}

// ---- Linear and PhiAttention (reference src/layer.cu:21-42, 150-188) --------

Linear::Linear(Tensor weight, Tensor bias) : weight_(std::move(weight)), bias_(std::move(bias)) {
    if (weight_.ndim() != 2 || (bias_.size() && bias_.size() != weight_.size(0)))
        throw std::invalid_argument("Linear weight shapes");
}

Linear::Linear(const ModelLoader& loader, const std::string& weight, const std::string& bias)
    : Linear(loader.load(weight), bias.empty() ? Tensor() : loader.load(bias)) {}

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
    (void)seq_lens;  // the trie path takes positions and key chains from the expansion
    if (!use_gpu) throw std::invalid_argument("PhiAttention::forward: the CPU path (use_gpu = false) is not provided");
    if (!expansion.active() || !expansion.node_pos)
        throw std::invalid_argument("PhiAttention::forward: this build provides the prefix-trie path (an active expansion)");
    const std::size_t s = x.size(0);
    Tensor q, k, v;
    q_proj_.forward(x, q, true);
    k_proj_.forward(x, k, true);
    v_proj_.forward(x, v, true);
    tensor_ops::apply_rope_tree_gpu(q, k, expansion.node_pos->data(), s, expansion.max_seq,
                                    apss26::NUM_ATTENTION_HEADS, apss26::NUM_KV_HEADS, apss26::HEAD_DIM,
                                    apss26::ROPE_THETA);
    Tensor out({s, apss26::NUM_ATTENTION_HEADS * apss26::HEAD_DIM});
    tensor_ops::attention_tree_gpu(q, k, v, out, expansion.node_pos->data(), expansion.node_anc->data(),
                                   expansion.anc_stride, s, expansion.max_seq, apss26::NUM_ATTENTION_HEADS,
                                   apss26::NUM_KV_HEADS, apss26::HEAD_DIM);
    o_proj_.forward(out, y, true);
}
