// Test and benchmark driver of the C++ drop-in model: a C ABI over
// PhiTinyMoEModel (include/model.h) for callers that hold the weights on the
// device already (the Python tests and bench.py --host cpp).  The model is
// built from parts, as a reference caller without a model.bin would build
// it: every tensor is a Tensor of the reference's shape whose device copy is
// filled device-to-device from the caller's buffer, then
// PhiTinyMoEModel::generate() (the reference harness's timed call,
// src/main.cpp:585-594) runs on the prompts.
//
//   void* md_model_create(layers, hidden, vocab, experts, ffn, q_out, kv_out,
//                         n, names, dev_ptrs, moe_compute)
//       names[i] / dev_ptrs[i]: fp32 device buffers by the reference's
//       tensor names (model.embed_tokens.weight, model.layers.<i>.*, ...);
//       null on error (md_last_error()).
//   int md_generate(model, ids, lens, batch, logits_dev, seconds_out)
//       logits [batch][vocab] fp32 copied to logits_dev; the wall time of
//       generate() (device synchronised on both sides) in *seconds_out.
//   void md_model_free(model)
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdint>
#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/model.h"

namespace {

thread_local std::string g_err;

struct Built {
    PhiTinyMoEModel model;
    std::size_t vocab;
};

Tensor from_device(const std::map<std::string, const float*>& w, const std::string& name,
                   std::vector<std::size_t> shape) {
    auto it = w.find(name);
    if (it == w.end()) throw std::invalid_argument("model_drive: missing tensor " + name);
    Tensor t(shape);
    if (hipMemcpy(t.cuda_data_write(), it->second, t.size() * sizeof(float), hipMemcpyDeviceToDevice) != hipSuccess)
        throw std::runtime_error("model_drive: hipMemcpy " + name);
    return t;
}

}  // namespace

extern "C" {

const char* md_last_error() { return g_err.c_str(); }

void* md_model_create(int layers, int hidden, int vocab, int experts, int ffn, int q_out, int kv_out, int n,
                      const char* const* names, const float* const* dev_ptrs, int moe_compute) {
    try {
        std::map<std::string, const float*> w;
        for (int i = 0; i < n; ++i) w[names[i]] = dev_ptrs[i];
        const std::size_t H = hidden, V = vocab, F = ffn;
        std::vector<PhiDecoderLayer> ls;
        ls.reserve(layers);
        for (int l = 0; l < layers; ++l) {
            const std::string p = "model.layers." + std::to_string(l) + ".";
            auto lin = [&](const std::string& nm, std::size_t out, std::size_t in) {
                return Linear(from_device(w, p + "self_attn." + nm + ".weight", {out, in}),
                              from_device(w, p + "self_attn." + nm + ".bias", {out}));
            };
            PhiAttention att(lin("q_proj", q_out, H), lin("k_proj", kv_out, H), lin("v_proj", kv_out, H),
                             lin("o_proj", H, q_out));
            const std::string m = p + "block_sparse_moe.";
            std::vector<PhiMLP> ex;
            for (int e = 0; e < experts; ++e) {
                const std::string x = m + "experts." + std::to_string(e) + ".";
                ex.emplace_back(from_device(w, x + "w1.weight", {F, H}), from_device(w, x + "w2.weight", {H, F}),
                                from_device(w, x + "w3.weight", {F, H}));
            }
            PhiMoE moe(from_device(w, m + "gate.weight", {static_cast<std::size_t>(experts), H}), std::move(ex),
                       static_cast<aps_dtype>(moe_compute));
            ls.emplace_back(from_device(w, p + "input_layernorm.weight", {H}),
                            from_device(w, p + "input_layernorm.bias", {H}),
                            from_device(w, p + "post_attention_layernorm.weight", {H}),
                            from_device(w, p + "post_attention_layernorm.bias", {H}), std::move(att), std::move(moe));
        }
        Linear head(from_device(w, "lm_head.weight", {V, H}), from_device(w, "lm_head.bias", {V}));
        return new Built{PhiTinyMoEModel(from_device(w, "model.embed_tokens.weight", {V, H}),
                                         from_device(w, "model.norm.weight", {H}),
                                         from_device(w, "model.norm.bias", {H}), std::move(head), std::move(ls)),
                         V};
    } catch (const std::exception& e) {
        g_err = e.what();
        return nullptr;
    }
}

int md_generate(void* model, const int* ids, const int* lens, int batch, float* logits_dev, double* seconds_out) {
    try {
        const Built* b = static_cast<const Built*>(model);
        std::vector<std::vector<int>> prompts(batch);
        for (int i = 0, at = 0; i < batch; at += lens[i], ++i) prompts[i].assign(ids + at, ids + at + lens[i]);
        Tensor logits;
        if (hipDeviceSynchronize() != hipSuccess) throw std::runtime_error("model_drive: sync");
        const auto t0 = std::chrono::steady_clock::now();
        b->model.generate(prompts, logits);
        if (hipDeviceSynchronize() != hipSuccess) throw std::runtime_error("model_drive: sync");
        const auto t1 = std::chrono::steady_clock::now();
        if (seconds_out) *seconds_out = std::chrono::duration<double>(t1 - t0).count();
        if (logits.size() != static_cast<std::size_t>(batch) * b->vocab)
            throw std::runtime_error("model_drive: logits shape");
        if (logits_dev && hipMemcpy(logits_dev, logits.cuda_data(), logits.size() * sizeof(float),
                                    hipMemcpyDeviceToDevice) != hipSuccess)
            throw std::runtime_error("model_drive: hipMemcpy logits");
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    }
}

void md_model_free(void* model) { delete static_cast<Built*>(model); }

}  // extern "C"
