// GPU check of the C++ host API (include/tensor.h, include/layer.h).
//
//   layer_check <out_dir> [<model.bin>]
//
// Builds a small synthetic MoE layer (16 experts, H = 512, F = 128, 96
// tokens), runs PhiMoE::forward in fp32 and bf16 compute and PhiMLP::forward
// (expert 0 as a dense FFN) on the GPU, and writes inputs and outputs as
// raw little-endian fp32 files into <out_dir> for tests/test_gpu_cpp_layer.py
// to compare with the CPU oracle.  It also checks, in process, the
// reference's exception types and messages, the Tensor host/device
// synchronisation rules, and the prompt prefix trie (a hand-worked batch)
// and row gather (both overloads) of include/prefix.h and include/tensor.h.  Exit status 0 means every in-process check passed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/layer.h"
#include "../../include/model.h"
#include "../../include/prefix.h"

namespace {

int g_failures = 0;

void expect(bool ok, const char* what) {
    if (!ok) {
        std::fprintf(stderr, "FAIL: %s\n", what);
        ++g_failures;
    }
}

template <class Ex, class Fn>
void expect_throw(Fn fn, const char* message, const char* what) {
    try {
        fn();
    } catch (const Ex& e) {
        if (message && std::string(e.what()) != message) {
            std::fprintf(stderr, "FAIL: %s: message \"%s\", want \"%s\"\n", what, e.what(), message);
            ++g_failures;
        }
        return;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "FAIL: %s: wrong exception type (%s)\n", what, e.what());
        ++g_failures;
        return;
    }
    std::fprintf(stderr, "FAIL: %s: no exception\n", what);
    ++g_failures;
}

// Deterministic normal samples (xorshift64* + Box-Muller).
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
    double uniform() {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        return ((s * 0x2545F4914F6CDD1Dull) >> 11) * (1.0 / 9007199254740992.0);
    }
    float normal(float sigma) {
        const double u1 = uniform() + 1e-300, u2 = uniform();
        return static_cast<float>(sigma * std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
    }
};

Tensor random_tensor(std::vector<std::size_t> shape, Rng& rng, float sigma) {
    Tensor t(std::move(shape));
    float* p = t.data();
    for (std::size_t i = 0; i < t.size(); ++i) p[i] = rng.normal(sigma);
    return t;
}

void write_raw(const std::string& dir, const char* name, const Tensor& t) {
    const std::string path = dir + "/" + name + ".f32";
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) throw std::runtime_error("cannot write " + path);
    std::fwrite(t.data(), sizeof(float), t.size(), f);
    std::fclose(f);
}

// Raw little-endian fields for hand-made model.bin files.
void put_u32(std::string& b, uint32_t v) { b.append(reinterpret_cast<const char*>(&v), 4); }
void put_u64(std::string& b, uint64_t v) { b.append(reinterpret_cast<const char*>(&v), 8); }
std::string write_file(const std::string& path, const std::string& bytes) {
    std::ofstream f(path, std::ios::binary);
    f.write(bytes.data(), static_cast<std::streamsize>(bytes.size()));
    return path;
}

// model.bin mode: PhiMoE(loader, 0) and PhiMLP(loader, <expert 0>) on the
// tensor "x" of the file, fp32 compute, outputs written for the oracle
// comparison; then the loader's error messages on hand-made files.
int loader_check(const std::string& dir, const std::string& model) {
    const ModelLoader loader(model);
    expect(loader.has("x") && !loader.has("nope"), "ModelLoader::has");
    const Tensor x = loader.load("x");
    const PhiMoE moe(loader, 0);
    Tensor y;
    moe.forward(x, y, true);
    const PhiMLP mlp(loader, "model.layers.0.block_sparse_moe.experts.0");
    Tensor ymlp;
    mlp.forward(x, ymlp, true);
    write_raw(dir, "loader_y", y);
    write_raw(dir, "loader_mlp_y", ymlp);
    // PhiAttention's trie path on the 64 nodes of a two-prompt batch (the
    // file's x rows are the node rows)
    {
        std::vector<int> p1(40), p2(44);
        for (int i = 0; i < 40; ++i) p1[i] = i + 1;
        for (int i = 0; i < 44; ++i) p2[i] = i < 20 ? i + 1 : i + 30;
        const PrefixTrie trie = build_prefix_trie({p1, p2});
        expect(trie.nodes() == x.size(0), "attention batch has one node per x row");
        const tensor_ops::RowIndexBuffer pos(trie.node_depth), anc(trie.node_anc);
        PrefixExpansion ex;
        ex.node_pos = &pos;
        ex.node_anc = &anc;
        ex.anc_stride = trie.max_len;
        ex.max_seq = trie.max_len;
        const PhiAttention attn(loader, 0);
        Tensor ya;
        attn.forward(x, ya, trie.seq_lens, true, ex);
        write_raw(dir, "loader_attn", ya);
        // the packed path needs seq_lens covering the rows
        expect_throw<std::invalid_argument>([&] { attn.forward(x, ya, {1, 2}, true); }, "packed sequence lengths",
                                            "attention packed lengths");
        // an expansion whose positions run past max_seq is refused on the host
        PrefixExpansion short_ex = ex;
        short_ex.max_seq = 3;
        expect_throw<std::invalid_argument>([&] { attn.forward(x, ya, trie.seq_lens, true, short_ex); },
                                            "PhiAttention prefix expansion", "expansion positions checked");
    }
    expect_throw<std::runtime_error>([&] { (void)loader.load("nope"); }, "missing tensor: nope", "missing tensor");
    const std::string nofile = dir + "/absent.bin";
    expect_throw<std::runtime_error>([&] { ModelLoader l(nofile); }, ("cannot open model: " + nofile).c_str(),
                                     "cannot open");
    const std::string trunc = write_file(dir + "/trunc.bin", std::string("\x01\x00", 2));
    expect_throw<std::runtime_error>([&] { ModelLoader l(trunc); }, "truncated model.bin", "truncated index");
    std::string b;
    put_u32(b, 2);
    put_u32(b, 1);
    b += "b";
    put_u32(b, 1);
    put_u32(b, 3);
    put_u64(b, 0);
    put_u64(b, 8);  // 3 elements but 8 bytes
    put_u32(b, 1);
    b += "t";
    put_u32(b, 1);
    put_u32(b, 4);
    put_u64(b, 4096);  // past the end of the file
    put_u64(b, 16);
    const ModelLoader bad(write_file(dir + "/bad.bin", b));
    expect_throw<std::runtime_error>([&] { (void)bad.load("b"); }, "tensor is not float32: b", "not float32");
    expect_throw<std::runtime_error>([&] { (void)bad.load("t"); }, "truncated tensor: t", "truncated tensor");
    std::printf("layer_check (model.bin): %d failure(s)\n", g_failures);
    return g_failures ? 1 : 0;
}

// The prompts of the model mode (tests/test_gpu_cpp_layer.py uses the same):
// shared prefixes, a prompt that is a prefix of another, a lone token.
const std::vector<std::vector<int>> kPrompts = {
    {5, 6, 7, 8, 9, 10}, {5, 6, 7, 1, 2}, {3, 4}, {5, 6, 7, 8, 11}, {5, 6, 7}, {9}};

// model mode: a two-layer PhiTinyMoEModel from the file's layers 0 and 1
// (the loader constructor reads NUM_LAYERS layers; this one is built from
// PhiDecoderLayer(loader, i) parts): generate() on kPrompts, forward() on
// the first prompt, generate_decode() for three tokens of the third, a
// two-layer decoder-layer forward() chain on the packed prompts, the
// elementwise tensor_ops, and the reference's error messages.
int model_check(const std::string& dir, const std::string& model) {
    const ModelLoader loader(model);
    std::vector<PhiDecoderLayer> layers;
    for (std::size_t i = 0; i < 2; ++i) layers.emplace_back(loader, i);
    const Linear head(loader, "lm_head.weight", "lm_head.bias");
    const Linear head_nobias(loader, "lm_head.weight", "lm_head.no_such_bias");
    expect(head.bias().size() == head.weight().size(0), "lm_head bias loaded");
    expect(head_nobias.bias().size() == 0, "an absent bias is skipped, as the reference does");
    const PhiTinyMoEModel m(loader.load("model.embed_tokens.weight"), loader.load("model.norm.weight"),
                            loader.load("model.norm.bias"), head, std::move(layers));
    expect(m.num_layers() == 2, "two layers");
    Tensor gen;
    m.generate(kPrompts, gen);
    expect(gen.ndim() == 2 && gen.size(0) == kPrompts.size() && gen.size(1) == head.weight().size(0),
           "generate logits shape");
    write_raw(dir, "gen_logits", gen);
    Tensor fwd;
    m.forward(kPrompts[0], fwd, true);
    expect(fwd.ndim() == 2 && fwd.size(0) == 1, "forward logits shape");
    write_raw(dir, "fwd_logits", fwd);
    Tensor dec;
    std::vector<std::vector<int>> ids;
    m.generate_decode({kPrompts[2]}, 3, dec, ids);
    expect(dec.size(0) == 1 && dec.size(1) == 3 && ids.size() == 1 && ids[0].size() == 3, "decode shapes");
    write_raw(dir, "dec_logits", dec);
    Tensor idt({3});
    for (std::size_t i = 0; i < 3; ++i) idt.at(i) = static_cast<float>(ids[0][i]);
    write_raw(dir, "dec_ids", idt);
    expect_throw<std::runtime_error>([&] { Tensor l; m.generate({}, l); }, "generate received an empty input batch",
                                     "generate: empty batch");
    expect_throw<std::invalid_argument>([&] { Tensor l; m.forward({}, l, true); }, "empty input", "forward: empty");
    expect_throw<std::invalid_argument>([&] { Tensor l; m.forward({1, 32064}, l, true); }, "token out of vocabulary",
                                        "forward: token range");
    expect_throw<std::invalid_argument>([&] { Tensor l; m.forward({1}, l, false); }, nullptr, "forward: CPU path");
    expect_throw<std::runtime_error>([&] { Tensor l; std::vector<std::vector<int>> g; m.generate_decode({}, 2, l, g); },
                                     "generate_decode received an empty input batch", "decode: empty batch");
    expect_throw<std::invalid_argument>(
        [&] { Tensor l; std::vector<std::vector<int>> g; m.generate_decode({{1}}, 0, l, g); },
        "max_new_tokens must be positive", "decode: zero tokens");

    // the decoder layer's forward() on the packed prompts (no trie)
    {
        std::vector<std::size_t> lens, rows;
        for (const auto& p : kPrompts) {
            lens.push_back(p.size());
            for (int t : p) rows.push_back(static_cast<std::size_t>(t));
        }
        const Tensor emb = loader.load("model.embed_tokens.weight");
        Tensor h({rows.size(), emb.size(1)});
        tensor_ops::gather_rows_gpu(emb, rows, h);
        const PhiDecoderLayer l0(loader, 0), l1(loader, 1);
        Tensor a, b;
        l0.forward(h, a, lens, true);
        l1.forward(a, b, lens, true);
        write_raw(dir, "packed_layers", b);
        std::vector<std::size_t> bad = lens;
        bad.back() += 1;
        expect_throw<std::invalid_argument>([&] { Tensor c; l0.forward(h, c, bad, true); }, "packed sequence lengths",
                                            "packed lengths must cover the rows");
    }

    // elementwise ops and the paired projections
    {
        Rng rng(77);
        const std::size_t n = 6, c = 40;
        Tensor a = random_tensor({n, c}, rng, 1.0f), b = random_tensor({n, c}, rng, 1.0f);
        Tensor bias = random_tensor({c}, rng, 1.0f);
        write_raw(dir, "ew_a", a);
        write_raw(dir, "ew_b", b);
        write_raw(dir, "ew_bias", bias);
        Tensor s = a;
        tensor_ops::add_inplace_gpu(s, b);
        write_raw(dir, "ew_add", s);
        Tensor t = a;
        tensor_ops::add_bias_inplace_gpu(t, bias);
        write_raw(dir, "ew_add_bias", t);
        Tensor u({n, c});
        tensor_ops::silu_mul_gpu(a, b, u);
        write_raw(dir, "ew_silu_mul", u);
        Tensor z = a;
        tensor_ops::zero_gpu(z);
        bool zero = true;
        for (std::size_t i = 0; i < z.size(); ++i) zero = zero && z[i] == 0.0f;
        expect(zero, "zero_gpu");
        Tensor wrong({n, c + 1});
        expect_throw<std::invalid_argument>([&] { tensor_ops::add_inplace_gpu(s, wrong); }, "add shape", "add shape");
        expect_throw<std::invalid_argument>([&] { tensor_ops::add_bias_inplace_gpu(s, b); }, "bias shape", "bias shape");
        expect_throw<std::invalid_argument>([&] { tensor_ops::silu_mul_gpu(a, wrong, u); }, "silu_mul shape",
                                            "silu_mul shape");
        // matmul_pair_silu_gpu / matmul_pair_bias_gpu on the layer-0 expert 0 and k/v weights
        const std::string e0 = "model.layers.0.block_sparse_moe.experts.0.";
        const Tensor w1 = loader.load(e0 + "w1.weight"), w3 = loader.load(e0 + "w3.weight");
        const Tensor xin = random_tensor({n, w1.size(1)}, rng, 1.0f);
        write_raw(dir, "pair_x", xin);
        Tensor ps({n, w1.size(0)});
        tensor_ops::matmul_pair_silu_gpu(xin, w1, w3, ps);
        write_raw(dir, "pair_silu", ps);
        const Tensor kw = loader.load("model.layers.0.self_attn.k_proj.weight");
        const Tensor kb = loader.load("model.layers.0.self_attn.k_proj.bias");
        const Tensor vw = loader.load("model.layers.0.self_attn.v_proj.weight");
        const Tensor vb = loader.load("model.layers.0.self_attn.v_proj.bias");
        Tensor ko({n, kw.size(0)}), vo({n, vw.size(0)});
        tensor_ops::matmul_pair_bias_gpu(xin, kw, kb, ko, vw, vb, vo);
        write_raw(dir, "pair_k", ko);
        write_raw(dir, "pair_v", vo);
        Tensor bad({n, w1.size(0) + 4});
        expect_throw<std::invalid_argument>([&] { tensor_ops::matmul_pair_silu_gpu(xin, w1, w3, bad); },
                                            "matmul_pair_silu_gpu shape", "pair silu shape");
        expect_throw<std::invalid_argument>([&] { tensor_ops::matmul_pair_bias_gpu(xin, kw, kb, bad, vw, vb, vo); },
                                            "matmul_pair_bias_gpu shape", "pair bias shape");
    }
    std::printf("layer_check (model): %d failure(s)\n", g_failures);
    return g_failures ? 1 : 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2 || argc > 4) {
        std::fprintf(stderr, "usage: %s <out_dir> [<model.bin> [model]]\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    if (argc == 4) return model_check(dir, argv[2]);
    if (argc == 3) return loader_check(dir, argv[2]);
    const std::size_t T = 96, H = 512, F = 128, E = apss26::NUM_EXPERTS;
    Rng rng(20260);

    Tensor x = random_tensor({T, H}, rng, 1.0f);
    Tensor gate = random_tensor({E, H}, rng, 0.02f);
    std::vector<PhiMLP> experts;
    Tensor w1_all({E, F, H}), w2_all({E, H, F}), w3_all({E, F, H});
    for (std::size_t e = 0; e < E; ++e) {
        Tensor w1 = random_tensor({F, H}, rng, 0.02f);
        Tensor w2 = random_tensor({H, F}, rng, 0.02f);
        Tensor w3 = random_tensor({F, H}, rng, 0.02f);
        std::memcpy(w1_all.data() + e * F * H, w1.data(), F * H * sizeof(float));
        std::memcpy(w2_all.data() + e * H * F, w2.data(), H * F * sizeof(float));
        std::memcpy(w3_all.data() + e * F * H, w3.data(), F * H * sizeof(float));
        experts.emplace_back(std::move(w1), std::move(w2), std::move(w3));
    }

    // --- MoE block, fp32 and bf16 compute -----------------------------------
    PhiMoE moe32(gate, experts, APS_DTYPE_F32);
    PhiMoE moe16(gate, experts, APS_DTYPE_BF16);
    Tensor y32, y16;
    moe32.forward(x, y32, true);
    moe16.forward(x, y16, true);
    expect(y32.ndim() == 2 && y32.size(0) == T && y32.size(1) == H, "PhiMoE output shape");
    expect(y16.size() == T * H, "PhiMoE bf16 output size");

    // --- dense FFN (expert 0 as PhiMLP) --------------------------------------
    Tensor x3 = x;
    x3.reshape({2, T / 2, H});
    Tensor ymlp;
    experts[0].forward(x3, ymlp, true);
    expect(ymlp.shape() == x3.shape(), "PhiMLP keeps the input shape");

    // --- router GEMM on its own ----------------------------------------------
    Tensor logits({T, E});
    tensor_ops::matmul_transposed_gpu(x, gate, logits);

    // --- decoder-layer LayerNorm: plain, and x += residual in place ----------
    Tensor ln_w = random_tensor({H}, rng, 1.0f), ln_b = random_tensor({H}, rng, 0.1f);
    Tensor resid = random_tensor({T, H}, rng, 1.0f);
    Tensor ln_y({T, H}), ln_x = x, add_y({T, H});
    tensor_ops::layer_norm_gpu(x, ln_w, ln_b, apss26::NORM_EPS, ln_y);
    tensor_ops::add_layer_norm_gpu(ln_x, resid, ln_w, ln_b, apss26::NORM_EPS, add_y);
    {
        Tensor bad({T, H - 1});
        expect_throw<std::invalid_argument>([&] { tensor_ops::layer_norm_gpu(x, ln_w, ln_b, 1e-5f, bad); },
                                            "layer norm shape", "layer norm shape");
        expect_throw<std::invalid_argument>(
            [&] { tensor_ops::add_layer_norm_gpu(ln_x, bad, ln_w, ln_b, 1e-5f, add_y); }, "add layer norm shape",
            "add layer norm shape");
    }

    // --- prompt prefix dedup and the row gather --------------------------------
    {
        const PrefixTrie trie = build_prefix_trie({{1, 2, 3}, {1, 2, 4}, {5}, {1, 2, 3, 6}});
        expect(trie.token_node == std::vector<std::size_t>({0, 1, 2, 0, 1, 3, 4, 0, 1, 2, 5}), "trie token_node");
        expect(trie.node_token == std::vector<std::size_t>({1, 2, 3, 4, 5, 6}), "trie node_token");
        expect(trie.node_depth == std::vector<std::size_t>({0, 1, 2, 2, 0, 3}), "trie node_depth");
        expect(trie.max_len == 4 && trie.node_anc.size() == 6 * 4, "trie ancestor table size");
        expect(std::vector<std::size_t>(trie.node_anc.begin() + 20, trie.node_anc.end()) ==
                   std::vector<std::size_t>({0, 1, 2, 5}), "trie ancestor chain of node 5");
        expect(std::vector<std::size_t>(trie.node_anc.begin() + 16, trie.node_anc.begin() + 20) ==
                   std::vector<std::size_t>({4, 0, 0, 0}), "trie ancestor chain of node 4");
        expect(trie.last_rows() == std::vector<std::size_t>({2, 3, 4, 5}), "trie last rows");
        // the device-built table equals the host one, on this trie and on
        // branchier ones (tiny vocabularies, repeated and nested prompts)
        std::mt19937 trng(17);
        const std::vector<std::vector<std::vector<int>>> tries = {
            {{1, 2, 3}, {1, 2, 4}, {5}, {1, 2, 3, 6}},
            {std::vector<int>(50, 7), std::vector<int>(50, 7), std::vector<int>(9, 7), {7, 8}},
            [&] {
                std::vector<std::vector<int>> b(30);
                for (auto& q : b) {
                    q.resize(1 + trng() % 70);
                    for (int& tok : q) tok = static_cast<int>(trng() % 3);
                }
                return b;
            }()};
        for (const auto& batch : tries) {
            const PrefixTrie tt = build_prefix_trie(batch);
            const tensor_ops::RowIndexBuffer dev = prefix_ancestors_gpu(build_prefix_trie(batch, false));
            std::vector<std::uint32_t> got(dev.size());
            expect(hipMemcpy(got.data(), dev.data(), got.size() * 4, hipMemcpyDeviceToHost) == hipSuccess,
                   "copy device ancestor table");
            expect(got.size() == tt.node_anc.size() && std::equal(got.begin(), got.end(), tt.node_anc.begin()),
                   "prefix_ancestors_gpu equals the host ancestor table");
            expect(dev.max_row() == tt.nodes() - 1, "device ancestor table row bound");
        }
        expect_throw<std::runtime_error>([] { build_prefix_trie({}); }, "generate received an empty input batch",
                                         "empty batch");
        expect_throw<std::invalid_argument>([] { build_prefix_trie({{1}, {}}); }, "empty input", "empty sequence");
        expect_throw<std::invalid_argument>([] { build_prefix_trie({std::vector<int>(4097, 1)}); },
                                            "sequence is too long", "long sequence");
        expect_throw<std::invalid_argument>([] { build_prefix_trie({{1, 32064}}); }, "token out of vocabulary",
                                            "token range");
        // gather rows of x: the vector overload and a device index map
        const std::vector<std::size_t> rows = {T - 1, 0, 5, 5, 17};
        Tensor g1({rows.size(), H}), g2({rows.size(), H});
        tensor_ops::gather_rows_gpu(x, rows, g1);
        const tensor_ops::RowIndexBuffer rib(rows);
        tensor_ops::gather_rows_gpu(x, rib, g2);
        bool same = true;
        for (std::size_t i = 0; i < rows.size(); ++i)
            for (std::size_t k = 0; k < H; ++k)
                same = same && g1.at(i, k) == x.at(rows[i], k) && g2.at(i, k) == x.at(rows[i], k);
        expect(same, "gather_rows_gpu copies the indexed rows");
        Tensor g3({2, H});
        expect_throw<std::invalid_argument>([&] { tensor_ops::gather_rows_gpu(x, {0, T}, g3); },
                                            "gather_rows_gpu row index", "gather index past the end");
        expect_throw<std::invalid_argument>([&] { tensor_ops::gather_rows_gpu(x, {0, 1}, g1); },
                                            "gather_rows_gpu shape", "gather output size");
    }

    // --- tree attention on a small trie: RoPE, then attention ----------------
    {
        const PrefixTrie trie = build_prefix_trie({{5, 6, 7, 8, 9}, {5, 6, 7, 1}, {2, 3}});
        const std::size_t n = trie.nodes(), qh = apss26::NUM_ATTENTION_HEADS, kvh = apss26::NUM_KV_HEADS,
                          hd = apss26::HEAD_DIM;
        Tensor aq = random_tensor({n, qh * hd}, rng, 1.0f), ak = random_tensor({n, kvh * hd}, rng, 1.0f),
               av = random_tensor({n, kvh * hd}, rng, 1.0f);
        write_raw(dir, "attn_q", aq);
        write_raw(dir, "attn_k", ak);
        write_raw(dir, "attn_v", av);
        const tensor_ops::RowIndexBuffer pos(trie.node_depth), anc(trie.node_anc);
        tensor_ops::apply_rope_tree_gpu(aq, ak, pos.data(), n, apss26::MAX_POSITION_EMBEDDINGS, qh, kvh, hd,
                                        apss26::ROPE_THETA);
        Tensor ao({n, qh * hd});
        tensor_ops::attention_tree_gpu(aq, ak, av, ao, pos.data(), anc.data(), trie.max_len, n,
                                       apss26::MAX_POSITION_EMBEDDINGS, qh, kvh, hd);
        write_raw(dir, "attn_qr", aq);
        write_raw(dir, "attn_kr", ak);
        write_raw(dir, "attn_out", ao);
        expect_throw<std::invalid_argument>(
            [&] { tensor_ops::attention_tree_gpu(aq, ak, av, ao, pos.data(), anc.data(), trie.max_len, n, 4096, 16, 2,
                                                 hd); },
            "attention_tree_gpu expects GQA-4", "GQA-4 check");
    }

    // --- packed attention in another head layout (4 heads of 64, one KV
    //     head each): the reference's generic kernel -----------------------
    {
        const std::vector<std::size_t> lens = {5, 3, 1};
        const std::size_t rows = 9, heads = 4, hd = 64;
        Tensor pq = random_tensor({rows, heads * hd}, rng, 1.0f), pk = random_tensor({rows, heads * hd}, rng, 1.0f),
               pv = random_tensor({rows, heads * hd}, rng, 1.0f);
        write_raw(dir, "mha_q", pq);
        write_raw(dir, "mha_k", pk);
        write_raw(dir, "mha_v", pv);
        Tensor po({rows, heads * hd});
        tensor_ops::attention_gpu(pq, pk, pv, po, lens, heads, heads, hd);
        write_raw(dir, "mha_out", po);
    }

    // --- the split-bf16 Linear (Tensor::prepare_cuda_bf16_weight) ------------
    {
        const std::size_t m = 70, k = 256, n = 132;
        Tensor lx = random_tensor({m, k}, rng, 1.0f), lw = random_tensor({n, k}, rng, 0.05f),
               lb = random_tensor({n}, rng, 0.1f);
        Tensor y32({m, n}), ytc({m, n}), ytc0({m, n});
        tensor_ops::matmul_transposed_bias_gpu(lx, lw, lb, y32);
        Tensor lw_tc = lw;                       // a copy does not carry the bf16 images
        expect(!lw_tc.has_cuda_bf16_weight(), "fresh weight has no bf16 copy");
        lw_tc.prepare_cuda_bf16_weight(true);
        expect(lw_tc.has_cuda_bf16_weight() && lw_tc.cuda_bf16_weight_lo() != nullptr, "bf16 copy prepared");
        tensor_ops::matmul_transposed_bias_gpu(lx, lw_tc, lb, ytc);
        tensor_ops::matmul_transposed_gpu(lx, lw_tc, ytc0);
        double worst = 0.0, worst0 = 0.0;
        bool differs = false;
        for (std::size_t i = 0; i < m; ++i)
            for (std::size_t j = 0; j < n; ++j) {
                double sc = std::fabs(lb.at(j));
                for (std::size_t q = 0; q < k; ++q) sc += std::fabs(static_cast<double>(lx.at(i, q)) * lw.at(j, q));
                const double d = std::fabs(static_cast<double>(ytc.at(i, j)) - y32.at(i, j));
                const double d0 = std::fabs(static_cast<double>(ytc0.at(i, j)) + lb.at(j) - y32.at(i, j));
                worst = std::max(worst, d / sc);
                worst0 = std::max(worst0, d0 / sc);
                differs = differs || ytc.at(i, j) != y32.at(i, j);
            }
        expect(worst < 3e-5 && worst0 < 3e-5, "split-bf16 Linear within 3e-5 of the fp32 chain");
        expect(differs, "the split-bf16 path ran (results differ from the fp32 chain in some bits)");
        // the fp32 device copy was released after packing (as the reference);
        // the host copy is intact and a device read uploads it again
        bool host_same = true;
        for (std::size_t j = 0; j < n; ++j)
            for (std::size_t q = 0; q < k; ++q) host_same = host_same && lw_tc.at(j, q) == lw.at(j, q);
        expect(host_same, "host fp32 copy intact after packing");
        std::vector<float> back(n * k);
        expect(hipMemcpy(back.data(), lw_tc.cuda_data(), n * k * sizeof(float), hipMemcpyDeviceToHost) == hipSuccess,
               "hipMemcpy of the uploaded weight");
        bool dev_same = true;
        for (std::size_t j = 0; j < n; ++j)
            for (std::size_t q = 0; q < k; ++q) dev_same = dev_same && back[j * k + q] == lw.at(j, q);
        expect(dev_same, "fp32 device copy uploaded again after packing");
        Tensor moved = std::move(lw_tc);
        expect(moved.has_cuda_bf16_weight() && !lw_tc.has_cuda_bf16_weight(), "a move carries the bf16 copy");
        Tensor v3({4});
        expect_throw<std::invalid_argument>([&] { v3.prepare_cuda_bf16_weight(true); },
                                            "BF16 packing requires a matrix", "bf16 packing of a vector");
    }

    // --- Tensor synchronisation rules ----------------------------------------
    {
        Tensor t({4, 8});
        t.fill(2.0f);
        const float* d = t.cuda_data();       // upload
        expect(d != nullptr, "cuda_data uploads");
        float* w = t.cuda_data_write();       // device copy becomes the valid one
        expect(hipMemset(w, 0, 32 * sizeof(float)) == hipSuccess, "device memset");
        expect(hipDeviceSynchronize() == hipSuccess, "device sync");
        expect(t.at(3, 7) == 0.0f, "host sees the device write after cuda_data_write");
        t.at(0, 0) = 5.0f;                    // host copy becomes the valid one
        const float* d2 = t.cuda_data();
        float back = 0.0f;
        expect(hipMemcpy(&back, d2, sizeof(float), hipMemcpyDeviceToHost) == hipSuccess, "readback");
        expect(back == 5.0f, "device sees the host write after a non-const at()");
        Tensor u = t;                         // deep copy of the host data
        u.at(0, 0) = 7.0f;
        expect(t.at(0, 0) == 5.0f, "copies are independent");
        expect_throw<std::out_of_range>([&] { (void)t.at(4, 0); }, "Tensor index", "at() bounds");
        expect_throw<std::invalid_argument>([&] { (void)t.at(1); }, "Tensor rank mismatch", "at() rank");
        expect_throw<std::out_of_range>([&] { (void)t.size(2); }, "Tensor dimension", "size(dim) bounds");
        expect_throw<std::invalid_argument>([&] { t.reshape({5, 7}); }, "reshape changes tensor size", "reshape");
        // a device-resident tensor copies on the device and stays independent
        Tensor dv({4, 8});
        float* dw = dv.cuda_data_write();
        std::vector<float> ramp(32);
        for (int i = 0; i < 32; ++i) ramp[i] = static_cast<float>(i);
        expect(hipMemcpy(dw, ramp.data(), sizeof(float) * 32, hipMemcpyHostToDevice) == hipSuccess, "ramp upload");
        Tensor dc = dv;
        Tensor moved = std::move(dc);
        dv.at(1, 1) = -1.0f;
        expect(moved.at(1, 1) == 9.0f && moved.at(3, 7) == 31.0f, "device copy then move keeps the values");
        expect(dv.at(1, 1) == -1.0f && dv.at(3, 7) == 31.0f, "source keeps its own values");
        // a fresh tensor reads as zeros on both sides
        Tensor fresh({3, 5});
        const float* fz = fresh.cuda_data();
        float probe = 1.0f;
        expect(hipMemcpy(&probe, fz + 14, sizeof(float), hipMemcpyDeviceToHost) == hipSuccess && probe == 0.0f,
               "fresh tensor uploads zeros");
        expect(fresh.at(2, 4) == 0.0f, "fresh tensor reads zeros on the host");
        Tensor assigned({1});
        assigned = dv;
        expect(assigned.shape() == dv.shape() && assigned.at(3, 7) == 31.0f, "copy assignment");
    }

    // --- the reference's exceptions -------------------------------------------
    {
        std::vector<const Tensor*> w1, w2, w3;
        for (std::size_t e = 0; e + 1 < E; ++e) {
            w1.push_back(&experts[e].w1());
            w2.push_back(&experts[e].w2());
            w3.push_back(&experts[e].w3());
        }
        expect_throw<std::invalid_argument>([&] { tensor_ops::register_moe_weights_gpu(w1, w2, w3); },
                                            "MoE weight table size", "15-expert table");
        Tensor bad_router({T, E - 1}), out;
        expect_throw<std::invalid_argument>([&] { tensor_ops::moe_forward_grouped_gpu(x, bad_router, 1, out); },
                                            "grouped MoE shape or handle", "router shape");
        Tensor router({T, E});
        expect_throw<std::invalid_argument>([&] { tensor_ops::moe_forward_grouped_gpu(x, router, 0, out); },
                                            "grouped MoE shape or handle", "handle 0");
        expect_throw<std::invalid_argument>([&] { tensor_ops::moe_forward_grouped_gpu(x, router, 1u << 20, out); },
                                            "grouped MoE shape or handle", "unknown handle");
        Tensor c({T, 3});
        expect_throw<std::invalid_argument>([&] { tensor_ops::matmul_transposed_gpu(x, gate, c); },
                                            "matmul_transposed_gpu shape", "matmul shape");
        Tensor y;
        expect_throw<std::invalid_argument>([&] { moe32.forward(x, y, false); }, nullptr, "CPU path");
    }

    write_raw(dir, "x", x);
    write_raw(dir, "gate", gate);
    write_raw(dir, "w1", w1_all);
    write_raw(dir, "w2", w2_all);
    write_raw(dir, "w3", w3_all);
    write_raw(dir, "y_f32", y32);
    write_raw(dir, "y_bf16", y16);
    write_raw(dir, "mlp_y", ymlp);
    write_raw(dir, "logits", logits);
    write_raw(dir, "ln_w", ln_w);
    write_raw(dir, "ln_b", ln_b);
    write_raw(dir, "resid", resid);
    write_raw(dir, "ln_y", ln_y);
    write_raw(dir, "ln_x", ln_x);
    write_raw(dir, "add_y", add_y);
    std::printf("layer_check: %d failure(s)\n", g_failures);
    return g_failures ? 1 : 0;
}
