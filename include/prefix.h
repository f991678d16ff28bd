// Prefix deduplication of a prompt batch: the trie walk of the reference's
// PhiTinyMoEModel::generate (src/model.cu:44-117) as a free function, over
// the C ABI's aps_prefix_dedup (include/aps_moe.h).
//
// A token's hidden state depends only on the prefix that ends at it, so a
// layer's row-wise ops run once per trie node: gather the node rows with
// tensor_ops::gather_rows_gpu(embeddings, trie.node_token, hidden), run the
// layers on them, and read a prompt's last token at trie.last_rows().  Node
// ids, depths and ancestor chains are the reference's, in the same order.
#pragma once

#include <cstddef>
#include <vector>

#include "tensor.h"

struct PrefixTrie {
    std::vector<std::size_t> seq_lens;    // [batch]
    std::vector<std::size_t> offsets;     // [batch]: packed row of each sequence's first token
    std::vector<std::size_t> token_node;  // [total]: node of each packed token row
    std::vector<std::size_t> node_token;  // [nodes]: token id of each node
    std::vector<std::size_t> node_depth;  // [nodes]: depth = RoPE position
    std::vector<std::size_t> node_anc;    // [nodes][max_len]: chain root .. node, then zeros
    std::size_t max_len = 0;

    std::size_t nodes() const { return node_token.size(); }
    // node of each sequence's last token (reference src/model.cu:148-151)
    std::vector<std::size_t> last_rows() const;
};

// Throws std::runtime_error("generate received an empty input batch") for
// an empty batch and std::invalid_argument with the reference's messages
// ("empty input", "sequence is too long", "token out of vocabulary").
// with_ancestors = false leaves node_anc empty (prefix_ancestors_gpu builds
// the table on the device instead).
PrefixTrie build_prefix_trie(const std::vector<std::vector<int>>& input_ids, bool with_ancestors = true);

// The ancestor table [nodes][max_len] of a trie (node_anc's layout and
// values) built on the device by aps_prefix_ancestors from each node's
// parent, depth and run of consecutive ids: 12 bytes per node cross the bus
// instead of 4 x max_len.  Needs only token_node, node_depth, offsets and
// max_len, so a trie built without ancestors serves.  Synchronous.
tensor_ops::RowIndexBuffer prefix_ancestors_gpu(const PrefixTrie& trie);
