// Per-model runtime state shared by the model loader (model_llama2.cpp) and the fused executor (fused.cpp).
#pragma once
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "runtime.h"
#include "vkllm/vkllm_kvcache.h"
#include "vkllm/vkllm_models_llama2.h"

struct FusedState; // fused.cpp

struct ModelPriv
{
    // HBM layout: one slab holds every fp16 matrix. Per layer: [Wq; Wk; Wv] as one [3D, D] matrix, Wo [D, D],
    // [Wu; Wg] as one [2F, D] matrix (up rows first), Wd [D, F]; then the token embedding [V, D] and the output
    // matrix [V, D]. A second slab holds the fp32 norm weights.
    void *slab = nullptr;
    size_t slab_bytes = 0;
    void *norm_slab = nullptr;
    bool fused_ok = false; // every weight is fp16 in the slab with the shapes the fused kernels need

    uint32_t L = 0, D = 0, H = 0, hd = 0, F = 0, V = 0, ctx = 0;
    float eps = 1e-6f, theta = 10000.f;
    uint32_t pad_id = 0;

    struct Layer
    {
        uint16_t *wqkv, *wo, *wug, *wd;
        float *attn_norm, *ffn_norm;
        uint16_t *kc, *vc; // [H, ctx, hd]
    };
    std::vector<Layer> layers;
    uint16_t *embd = nullptr, *out_w = nullptr;
    float *out_norm = nullptr;
    std::vector<float> rope_freqs; // base^(2w/hd), host powf

    FusedState *fs = nullptr;
    std::unordered_map<std::string, int> vocab_index; // tokenizer lookups, first id of each text
};

inline ModelPriv *model_priv(vkllm_models_llama2 *m)
{
    return (ModelPriv *)m->priv;
}

// bind ModelPriv::layers[*].kc/vc to the model's KV cache tensors
void model_bind_kv(vkllm_context *ctx, vkllm_models_llama2 *model);
