// PhiTinyMoEModel (declared in include/model.h).  Reference:
// src/model.cu:10-204 -- the tensor names, generate()'s order of operations
// (trie, node-row gather, layers with the carried residual, final
// add+LayerNorm, last-row gather, LM head), forward()'s checks and messages,
// and generate_decode()'s greedy loop.
#include "../../include/model.h"

#include <stdexcept>
#include <utility>

#include "../../include/prefix.h"

namespace {

std::vector<PhiDecoderLayer> load_layers(const ModelLoader& loader, aps_dtype moe_compute) {
    std::vector<PhiDecoderLayer> layers;
    layers.reserve(apss26::NUM_LAYERS);
    for (std::size_t i = 0; i < apss26::NUM_LAYERS; ++i) layers.emplace_back(loader, i, moe_compute);
    return layers;
}

}  // namespace

PhiTinyMoEModel::PhiTinyMoEModel(const std::string& model_file, aps_dtype moe_compute)
    : loader_(std::make_unique<ModelLoader>(model_file)),
      embeddings_(loader_->load("model.embed_tokens.weight")),
      final_norm_weight_(loader_->load("model.norm.weight")),
      final_norm_bias_(loader_->load("model.norm.bias")),
      lm_head_(*loader_, "lm_head.weight", "lm_head.bias"),
      layers_(load_layers(*loader_, moe_compute)) {}

PhiTinyMoEModel::PhiTinyMoEModel(Tensor embeddings, Tensor final_norm_weight, Tensor final_norm_bias, Linear lm_head,
                                 std::vector<PhiDecoderLayer> layers)
    : embeddings_(std::move(embeddings)),
      final_norm_weight_(std::move(final_norm_weight)),
      final_norm_bias_(std::move(final_norm_bias)),
      lm_head_(std::move(lm_head)),
      layers_(std::move(layers)) {}

void PhiTinyMoEModel::generate(const std::vector<std::vector<int>>& input_ids, Tensor& logits) const {
    // validation and messages: the trie walk's (src/model.cu:47-117)
    const PrefixTrie trie = build_prefix_trie(input_ids, false);
    const std::size_t batch = input_ids.size(), hidden_size = embeddings_.size(1);

    // one row per trie node: the embedding rows of the node tokens
    Tensor hidden({trie.nodes(), hidden_size});
    tensor_ops::gather_rows_gpu(embeddings_, trie.node_token, hidden);
    // the ancestor table is nodes x max_len words: built on the device from
    // 12 bytes per node rather than filled on the host and uploaded
    const tensor_ops::RowIndexBuffer node_pos(trie.node_depth), node_anc(prefix_ancestors_gpu(trie));
    PrefixExpansion expansion;
    expansion.node_pos = &node_pos;
    expansion.node_anc = &node_anc;
    expansion.anc_stride = trie.max_len;
    expansion.max_seq = trie.max_len;

    Tensor carry;
    bool has_carry = false;
    for (const PhiDecoderLayer& layer : layers_) {
        layer.forward_carry(hidden, carry, has_carry, trie.seq_lens, expansion);
        has_carry = true;
    }
    // the last layer's residual add rides into the final norm
    Tensor normed(hidden.shape());
    if (has_carry)
        tensor_ops::add_layer_norm_gpu(hidden, carry, final_norm_weight_, final_norm_bias_, apss26::NORM_EPS, normed);
    else
        tensor_ops::layer_norm_gpu(hidden, final_norm_weight_, final_norm_bias_, apss26::NORM_EPS, normed);

    Tensor last({batch, hidden_size});
    tensor_ops::gather_rows_gpu(normed, trie.last_rows(), last);
    lm_head_.forward(last, logits, true);
    logits.reshape({batch, lm_head_.weight().size(0)});
}

void PhiTinyMoEModel::forward(const std::vector<int>& input_ids, Tensor& logits, bool use_gpu) const {
    if (!use_gpu)
        throw std::invalid_argument("PhiTinyMoEModel::forward: the CPU path (use_gpu = false) is not provided");
    if (input_ids.empty()) throw std::invalid_argument("empty input");
    const std::size_t s = input_ids.size(), hidden_size = embeddings_.size(1);
    if (s > apss26::MAX_POSITION_EMBEDDINGS) throw std::invalid_argument("sequence is too long");
    std::vector<std::size_t> rows(s);
    for (std::size_t i = 0; i < s; ++i) {
        const int token = input_ids[i];
        if (token < 0 || static_cast<std::size_t>(token) >= apss26::VOCAB_SIZE)
            throw std::invalid_argument("token out of vocabulary");
        rows[i] = static_cast<std::size_t>(token);
    }
    Tensor hidden({s, hidden_size});
    tensor_ops::gather_rows_gpu(embeddings_, rows, hidden);
    const std::vector<std::size_t> seq_lens{s};
    for (const PhiDecoderLayer& layer : layers_) {
        Tensor next;
        layer.forward(hidden, next, seq_lens, true);
        hidden = std::move(next);
    }
    Tensor normed(hidden.shape());
    tensor_ops::layer_norm_gpu(hidden, final_norm_weight_, final_norm_bias_, apss26::NORM_EPS, normed);
    Tensor last({1, hidden_size});
    tensor_ops::gather_rows_gpu(normed, std::vector<std::size_t>{s - 1}, last);
    lm_head_.forward(last, logits, true);
    logits.reshape({1, lm_head_.weight().size(0)});
}

void PhiTinyMoEModel::generate_decode(const std::vector<std::vector<int>>& input_ids, std::size_t max_new_tokens,
                                      Tensor& logits, std::vector<std::vector<int>>& generated_ids) const {
    if (input_ids.empty()) throw std::runtime_error("generate_decode received an empty input batch");
    if (max_new_tokens == 0) throw std::invalid_argument("max_new_tokens must be positive");
    const std::size_t batch = input_ids.size(), vocab = lm_head_.weight().size(0);
    logits = Tensor({batch, max_new_tokens, vocab});
    float* out = logits.data();
    generated_ids.assign(batch, {});
    for (std::size_t b = 0; b < batch; ++b) {
        std::vector<int> prefix = input_ids[b];
        for (std::size_t step = 0; step < max_new_tokens; ++step) {
            Tensor step_logits;
            forward(prefix, step_logits, true);
            const float* l = step_logits.data();
            // greedy: the first maximum wins
            std::size_t best = 0;
            for (std::size_t v = 1; v < vocab; ++v)
                if (l[v] > l[best]) best = v;
            std::copy(l, l + vocab, out + (b * max_new_tokens + step) * vocab);
            const int next = static_cast<int>(best);
            generated_ids[b].push_back(next);
            if (next == apss26::EOS_TOKEN_ID) break;
            prefix.push_back(next);
        }
    }
}
