// Model constants under the reference's names (include/config.h:5-27 of the
// reference: namespace apss26), the same values.
#pragma once

#include <cstddef>

namespace apss26 {
constexpr std::size_t NUM_LAYERS = 32;
constexpr std::size_t HIDDEN_SIZE = 4096;
constexpr std::size_t NUM_EXPERTS = 16;
constexpr std::size_t TOP_K = 2;
constexpr std::size_t EXPERT_INTERMEDIATE_SIZE = 448;
// Router scores are canonicalised to this grid before the deterministic
// top-2 selection; a later expert replaces the current best only if its
// score is larger by more than ROUTER_TIE_EPS.
constexpr float ROUTER_SCORE_QUANTUM = 1.0e-3f;
constexpr float ROUTER_TIE_EPS = 2.0e-2f;
// LayerNorm epsilon of the decoder layer (reference include/config.h:19).
constexpr float NORM_EPS = 1.0e-5f;
// Token ids and sequence lengths the prefix trie accepts (reference
// include/config.h:7, 16).
constexpr std::size_t VOCAB_SIZE = 32064;
constexpr std::size_t MAX_POSITION_EMBEDDINGS = 4096;
// Attention of the decoder layer (reference include/config.h:10-12, 17-18).
constexpr std::size_t NUM_ATTENTION_HEADS = 16;
constexpr std::size_t NUM_KV_HEADS = 4;
constexpr std::size_t HEAD_DIM = 128;
constexpr std::size_t SLIDING_WINDOW = 2047;
constexpr float ROPE_THETA = 10000.0f;
// Greedy decoding (reference include/config.h:20, 24-25): the end-of-text
// token and the default number of generated tokens.  ROUTER_JITTER_EPS is
// declared by the reference and read nowhere, here neither.
constexpr float ROUTER_JITTER_EPS = 0.01f;
constexpr std::size_t MAX_DECODE_TOKENS = 8;
constexpr int EOS_TOKEN_ID = 32000;
}  // namespace apss26
