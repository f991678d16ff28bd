// Prefix deduplication of a prompt batch (host code), and the device build of
// its ancestor table.
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

// ---------------------------------------------------------------------------
// The ancestor table on the device.  Node ids are creation order, so a node
// created right after its parent (the common case: a sequence's tokens past
// the point where it leaves every earlier sequence's prefix) is parent + 1,
// and a trie path is a few runs of consecutive ids: run_start[n] is the
// first node of n's run (n itself when parent(n) != n - 1 or n has depth 0),
// and within a run depth(s + i) = depth(s) + i.  The ancestor of n at depth
// d <= depth(n) is therefore s + (d - depth(s)) for the first run start s on
// the way up (s = run_start[n], then run_start[parent[s]], ..) with depth(s)
// <= d: as many steps as the path has branch points.  One thread per (node,
// depth) entry; entries past the node's depth are 0, as in the host table.
namespace {
__global__ void __launch_bounds__(256)
k_prefix_ancestors(const uint32_t* __restrict__ parent, const uint32_t* __restrict__ depth,
                   const uint32_t* __restrict__ run_start, int64_t nodes, int64_t stride, uint32_t* __restrict__ anc) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= nodes * stride) return;
    const int64_t n = i / stride;
    const uint32_t d = static_cast<uint32_t>(i - n * stride);
    uint32_t v = 0u;
    if (d <= depth[n]) {
        // indices clamped to the table for memory safety only (a consistent
        // trie never needs it); each step moves to a strictly shallower run,
        // so at most depth(n) steps
        const uint32_t last = static_cast<uint32_t>(nodes - 1);
        uint32_t s = run_start[n];
        s = s < last ? s : last;
        for (uint32_t guard = 0; d < depth[s] && guard <= depth[n]; ++guard) {
            uint32_t p = parent[s];
            p = p < last ? p : last;
            s = run_start[p];
            s = s < last ? s : last;
        }
        v = d >= depth[s] ? s + (d - depth[s]) : 0u;
        // an ancestor is created before its descendants: never above n, so
        // the table only names rows below the node count whatever the input
        v = v < static_cast<uint32_t>(n) ? v : static_cast<uint32_t>(n);
    }
    anc[i] = v;
}
}  // namespace

hipError_t launch_prefix_ancestors(const uint32_t* parent, const uint32_t* depth, const uint32_t* run_start,
                                   int64_t nodes, int64_t stride, uint32_t* anc, hipStream_t s) {
    if (nodes <= 0) return hipSuccess;
    if (stride <= 0 || stride > (int64_t(1) << 24) || nodes > (int64_t(1) << 38) / stride) return hipErrorInvalidValue;
    const int64_t n = nodes * stride;
    hipLaunchKernelGGL(k_prefix_ancestors, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, s, parent,
                       depth, run_start, nodes, stride, anc);
    return hipGetLastError();
}

}  // namespace aps
