// build_prefix_trie over the C ABI's aps_prefix_dedup (declared in
// include/prefix.h).  Reference: PhiTinyMoEModel::generate,
// src/model.cu:44-117 (validation, trie walk, node numbering).
#include "../../include/prefix.h"

#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "../../include/aps_moe.h"
#include "../../include/config.h"

std::vector<std::size_t> PrefixTrie::last_rows() const {
    std::vector<std::size_t> r(seq_lens.size());
    for (std::size_t b = 0; b < seq_lens.size(); ++b) r[b] = token_node[offsets[b] + seq_lens[b] - 1];
    return r;
}

PrefixTrie build_prefix_trie(const std::vector<std::vector<int>>& input_ids) {
    if (input_ids.empty()) throw std::runtime_error("generate received an empty input batch");
    PrefixTrie t;
    const std::size_t batch = input_ids.size();
    t.seq_lens.resize(batch);
    t.offsets.resize(batch);
    std::vector<int64_t> seq_offsets(batch + 1, 0);
    for (std::size_t b = 0; b < batch; ++b) {
        t.seq_lens[b] = input_ids[b].size();
        t.offsets[b] = static_cast<std::size_t>(seq_offsets[b]);
        seq_offsets[b + 1] = seq_offsets[b] + static_cast<int64_t>(input_ids[b].size());
        t.max_len = std::max(t.max_len, input_ids[b].size());
    }
    const std::size_t total = static_cast<std::size_t>(seq_offsets[batch]);
    std::vector<int32_t> ids;
    ids.reserve(total);
    for (const auto& s : input_ids) ids.insert(ids.end(), s.begin(), s.end());
    std::vector<uint32_t> token_node(total ? total : 1), node_token(total ? total : 1), node_depth(total ? total : 1);
    // the ancestor table only when every length is valid (else the call fails on the lengths first)
    const bool with_anc = t.max_len > 0 && t.max_len <= apss26::MAX_POSITION_EMBEDDINGS;
    std::vector<uint32_t> anc(with_anc ? (total ? total : 1) * t.max_len : 0);
    int64_t nodes = 0;
    const int rc = aps_prefix_dedup(ids.data(), seq_offsets.data(), static_cast<int64_t>(batch),
                                    static_cast<int64_t>(apss26::VOCAB_SIZE),
                                    static_cast<int64_t>(apss26::MAX_POSITION_EMBEDDINGS), token_node.data(),
                                    node_token.data(), node_depth.data(), with_anc ? anc.data() : nullptr,
                                    static_cast<int64_t>(t.max_len ? t.max_len : 1), &nodes);
    if (rc == APS_ERR_ARG) throw std::invalid_argument(aps_moe_last_error());
    if (rc) throw std::runtime_error(aps_moe_last_error());
    const std::size_t n = static_cast<std::size_t>(nodes);
    t.token_node.assign(token_node.begin(), token_node.begin() + static_cast<std::ptrdiff_t>(total));
    t.node_token.assign(node_token.begin(), node_token.begin() + static_cast<std::ptrdiff_t>(n));
    t.node_depth.assign(node_depth.begin(), node_depth.begin() + static_cast<std::ptrdiff_t>(n));
    t.node_anc.assign(anc.begin(), anc.begin() + static_cast<std::ptrdiff_t>(n * t.max_len));
    return t;
}
