// Prefix deduplication of a prompt batch (host code).
//
// Reference: PhiTinyMoEModel::generate (src/model.cu:44-117).  Attention is
// causal and the sequences are independent, so a token's hidden state is a
// function of the prefix that ends at it; every row-wise op (LayerNorm, the
// projections, the MoE block) therefore runs once per node of the prompts'
// prefix trie instead of once per token.  The walk assigns node ids in
// creation order (sequence by sequence, position by position), records
// each node's token and depth (its RoPE position) and, when asked, its
// ancestor chain root .. node (the keys its causal attention sees), and maps
// every packed token row to its node.  Same node numbering and the same
// validation order as the reference, so the deduplicated row order is
// identical.
//
// The trie is a hash map from (parent, token) to child, as in the reference
// (key (parent + 1) << 32 | token, the virtual root being parent ~0).
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.hpp"

namespace aps {

int prefix_dedup(const int32_t* ids, const int64_t* seq_offsets, int64_t batch, int64_t vocab, int64_t max_positions,
                 uint32_t* token_node, uint32_t* node_token, uint32_t* node_depth, uint32_t* node_anc,
                 int64_t anc_stride, int64_t* nodes_out, std::string& err) {
    if (seq_offsets[0] != 0) {
        err = "sequence offsets must start at 0";
        return 2;
    }
    // lengths first, all of them, as the reference (src/model.cu:55-62)
    int64_t max_len = 0;
    for (int64_t b = 0; b < batch; ++b) {
        const int64_t len = seq_offsets[b + 1] - seq_offsets[b];
        if (len < 0) {
            err = "sequence offsets must not decrease";
            return 2;
        }
        if (len == 0) {
            err = "empty input";
            return 1;
        }
        if (len > max_positions) {
            err = "sequence is too long";
            return 1;
        }
        max_len = len > max_len ? len : max_len;
    }
    if (node_anc && anc_stride < max_len) {
        err = "ancestor stride shorter than the longest sequence";
        return 2;
    }
    const int64_t total = seq_offsets[batch] - seq_offsets[0];
    if (total > 0xFFFFFFFEll) {
        err = "batch too large for 32-bit node ids";
        return 2;
    }
    std::unordered_map<uint64_t, uint32_t> children;
    children.reserve(static_cast<size_t>(2 * total));
    std::vector<uint32_t> chain(static_cast<size_t>(max_len));
    uint32_t nodes = 0;
    for (int64_t b = 0; b < batch; ++b) {
        uint32_t parent = 0xFFFFFFFFu;  // virtual root
        const int64_t len = seq_offsets[b + 1] - seq_offsets[b];
        for (int64_t si = 0; si < len; ++si) {
            const int64_t row = seq_offsets[b] + si;
            const int32_t token = ids[row];
            if (token < 0 || token >= vocab) {
                err = "token out of vocabulary";
                return 1;
            }
            const uint64_t key = (static_cast<uint64_t>(parent + 1u) << 32) | static_cast<uint32_t>(token);
            const auto ins = children.emplace(key, nodes);
            uint32_t node = ins.first->second;
            if (ins.second) {  // a new node
                node_token[node] = static_cast<uint32_t>(token);
                node_depth[node] = static_cast<uint32_t>(si);
                chain[static_cast<size_t>(si)] = node;
                if (node_anc) {
                    uint32_t* anc = node_anc + static_cast<int64_t>(node) * anc_stride;
                    std::memcpy(anc, chain.data(), static_cast<size_t>(si + 1) * sizeof(uint32_t));
                    std::memset(anc + si + 1, 0, static_cast<size_t>(anc_stride - si - 1) * sizeof(uint32_t));
                }
                ++nodes;
            } else {
                chain[static_cast<size_t>(si)] = node;
            }
            token_node[row] = node;
            parent = node;
        }
    }
    *nodes_out = nodes;
    return 0;
}

}  // namespace aps
