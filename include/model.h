// The whole model (reference include/model.h:7-27, src/model.cu:10-204): the
// embedding table, NUM_LAYERS decoder layers, the final LayerNorm and the LM
// head, with the reference's prefill entry point generate().
//
// generate() packs the batch, collapses it onto the prefix trie of the
// prompts (one row per distinct prefix: build_prefix_trie), gathers the
// embedding rows of the trie nodes on the GPU, runs every layer's
// forward_carry on the node rows (attention over ancestor chains), folds the
// last residual into the final LayerNorm, gathers each prompt's last row and
// applies the LM head: logits [batch][vocab].  forward() runs one sequence
// through the packed path (no trie); generate_decode() is the reference's
// greedy loop over forward().  All computation is on the GPU: use_gpu =
// false (the reference's CPU path) throws std::invalid_argument.
#pragma once

#include <cstddef>
#include <memory>
#include <string>
#include <vector>

#include "layer.h"

class PhiTinyMoEModel {
public:
    // model.embed_tokens.weight, model.norm.{weight,bias}, lm_head.{weight,
    // bias} (the bias only if the file holds it) and model.layers.<i>.* for
    // i < NUM_LAYERS.  moe_compute picks the expert FFN kernels of every
    // layer (APS_DTYPE_F32: the reference's arithmetic; APS_DTYPE_BF16).
    explicit PhiTinyMoEModel(const std::string& model_file, aps_dtype moe_compute = APS_DTYPE_F32);
    // A model from its parts (any layer count), for callers without a model.bin.
    PhiTinyMoEModel(Tensor embeddings, Tensor final_norm_weight, Tensor final_norm_bias, Linear lm_head,
                    std::vector<PhiDecoderLayer> layers);

    // logits [1][vocab] of the last token of one sequence.
    void forward(const std::vector<int>& input_ids, Tensor& logits, bool use_gpu = false) const;
    // logits [batch][vocab] of each prompt's last token (the timed prefill).
    void generate(const std::vector<std::vector<int>>& input_ids, Tensor& logits) const;
    // Greedy decoding: up to max_new_tokens per prompt, stopping after
    // EOS_TOKEN_ID; logits [batch][max_new_tokens][vocab] (rows of steps
    // not taken stay zero).
    void generate_decode(const std::vector<std::vector<int>>& input_ids, std::size_t max_new_tokens, Tensor& logits,
                         std::vector<std::vector<int>>& generated_ids) const;

    std::size_t num_layers() const { return layers_.size(); }

private:
    std::unique_ptr<ModelLoader> loader_;  // null for a model built from parts
    Tensor embeddings_;
    Tensor final_norm_weight_, final_norm_bias_;
    Linear lm_head_;
    std::vector<PhiDecoderLayer> layers_;
};
