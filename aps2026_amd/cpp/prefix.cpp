// build_prefix_trie over the C ABI's aps_prefix_dedup (declared in
// include/prefix.h).  Reference: PhiTinyMoEModel::generate,
// src/model.cu:44-117 (validation, trie walk, node numbering).
#include "../../include/prefix.h"

#include <hip/hip_runtime.h>

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

PrefixTrie build_prefix_trie(const std::vector<std::vector<int>>& input_ids, bool with_ancestors) {
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
    const bool with_anc = with_ancestors && t.max_len > 0 && t.max_len <= apss26::MAX_POSITION_EMBEDDINGS;
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
    if (with_anc) t.node_anc.assign(anc.begin(), anc.begin() + static_cast<std::ptrdiff_t>(n * t.max_len));
    return t;
}

tensor_ops::RowIndexBuffer prefix_ancestors_gpu(const PrefixTrie& t) {
    const std::size_t n = t.nodes();
    if (n == 0 || t.max_len == 0) return tensor_ops::RowIndexBuffer();
    // parent of a node = the node of the previous token of any sequence
    // through it (all agree: a node is one prefix); a run starts where the
    // parent is not the previous id
    std::vector<std::size_t> parent(n, 0), run_start(n, 0);
    for (std::size_t b = 0; b < t.seq_lens.size(); ++b)
        for (std::size_t i = 1; i < t.seq_lens[b]; ++i)
            parent[t.token_node[t.offsets[b] + i]] = t.token_node[t.offsets[b] + i - 1];
    for (std::size_t v = 0; v < n; ++v)
        run_start[v] = (t.node_depth[v] == 0 || parent[v] + 1 != v) ? v : run_start[v - 1];
    const tensor_ops::RowIndexBuffer parent_d(parent), depth_d(t.node_depth), run_d(run_start);
    // every entry of row v is at most v (the kernel guarantees it)
    tensor_ops::RowIndexBuffer anc = tensor_ops::RowIndexBuffer::allocate(n * t.max_len, n - 1);
    const int rc = aps_prefix_ancestors(parent_d.data(), depth_d.data(), run_d.data(), static_cast<int64_t>(n),
                                        static_cast<int64_t>(t.max_len), anc.mutable_data(), nullptr);
    if (rc) throw std::runtime_error(aps_moe_last_error());
    // the inputs are freed on return: wait for the kernel first
    const hipError_t e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) throw std::runtime_error(std::string("prefix ancestors: ") + hipGetErrorString(e));
    return anc;
}
