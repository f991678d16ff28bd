"""Random-init Phi-tiny-MoE-shaped weights drawn on the device, keyed by the
reference's model.bin tensor names (test infrastructure)."""
import torch


def random_model_weights(device, H=4096, F=448, E=16, V=32064, layers=32, seed=5):
    """name -> fp32 device tensor: linear and expert weights, projection and
    LM-head biases ~N(0, 0.02), LayerNorm weight 1 and bias 0, embeddings
    ~N(0, 1), drawn in a fixed order from one seeded generator."""
    g = torch.Generator(device=device).manual_seed(seed)
    rn = lambda *shape, s=0.02: (s * torch.randn(shape, generator=g, device=device)).contiguous()
    W = {"model.embed_tokens.weight": rn(V, H, s=1.0), "model.norm.weight": torch.ones(H, device=device),
         "model.norm.bias": torch.zeros(H, device=device), "lm_head.weight": rn(V, H), "lm_head.bias": rn(V)}
    for i in range(layers):
        p = f"model.layers.{i}."
        for nm in ("input_layernorm", "post_attention_layernorm"):
            W[p + nm + ".weight"] = torch.ones(H, device=device)
            W[p + nm + ".bias"] = torch.zeros(H, device=device)
        for nm, (o, k) in (("q_proj", (2048, H)), ("k_proj", (512, H)), ("v_proj", (512, H)),
                           ("o_proj", (H, 2048))):
            W[p + f"self_attn.{nm}.weight"] = rn(o, k)
            W[p + f"self_attn.{nm}.bias"] = rn(o)
        m = p + "block_sparse_moe."
        W[m + "gate.weight"] = rn(E, H)
        for e in range(E):
            W[m + f"experts.{e}.w1.weight"] = rn(F, H)
            W[m + f"experts.{e}.w3.weight"] = rn(F, H)
            W[m + f"experts.{e}.w2.weight"] = rn(H, F)
    return W
