/* LLaMA-2 model: GGUF load, per-step graph, tokenizer. Replaces src/models/vkllm_models_llama2.h:6-146
 * (same structs, fields and functions; `priv` added for the HIP runtime's per-model state). */
#ifndef VKLLM_MODELS_LLAMA2_H
#define VKLLM_MODELS_LLAMA2_H
#include <stdbool.h>
#include <stdint.h>
#include "vkllm_array.h"
#include "vkllm_llama2_layers.h"
#ifdef __cplusplus
extern "C" {
#endif

struct block_weights
{
    struct vkllm_tensor *attn_norm_weight;
    struct vkllm_tensor *ffn_norm_weight;
    struct vkllm_tensor *WQ;
    struct vkllm_tensor *WK;
    struct vkllm_tensor *WV;
    struct vkllm_tensor *WO;
    struct vkllm_tensor *WU;
    struct vkllm_tensor *WG;
    struct vkllm_tensor *WD;
};

VKLLM_DEF_ARRAY(block_weights, struct block_weights *)

struct vkllm_graph;
struct vkllm_kvcache;

struct vkllm_token
{
    char *text;
    float score;
    int32_t type;
};

VKLLM_DEF_ARRAY(token, struct vkllm_token)
VKLLM_DEF_ARRAY(token_id, uint32_t)

struct vkllm_models_llama2
{
    struct
    {
        uint32_t block_count;
        uint32_t context_length;
        uint32_t embedding_length;
        float rope_freq_base;
        float layer_norm_rms_epsilon;
        uint32_t key_length;
        uint32_t value_length;
        uint32_t vocab_size;
        uint32_t head_count;
        uint32_t head_count_kv;
        uint32_t bos_token_id;
        uint32_t eos_token_id;
        uint32_t padding_token_id;
        bool add_bos_token;
        bool add_eos_token;
        struct vkllm_array_token *tokens;
    } meta;

    struct
    {
        struct vkllm_tensor *tok_embed_weights;
        struct vkllm_array_block_weights *blocks;
        struct vkllm_tensor *output_norm_weight;
        struct vkllm_tensor *output_weight;
        struct vkllm_kvcache *kvcache;
    } weights;

    void *priv; /* HIP runtime state: weight slabs, fused-plan buffers, captured decode graph */
};

/* src/models/vkllm_models_llama2.c:255-412: GGUF v3 file; missing keys take the reference's defaults
 * (src/models/vkllm_models_llama2.c:224-241); unreadable file -> VKLLM_ERR_ARGS */
extern vkllm_err_t vkllm_models_llama2_load(struct vkllm_context *context, struct vkllm_models_llama2 *model,
                                            const char *file);
extern vkllm_err_t vkllm_models_llama2_free(struct vkllm_context *context, struct vkllm_models_llama2 *model);
/* src/models/vkllm_models_llama2.c:488-602: adds input_toks [1,1,1,S] (uint32, mapped) and the step's nodes to
 * `graph`; output node = ARG_MAX [1,1,S,1] uint32 mapped. Frees the graph on failure. */
extern vkllm_err_t vkllm_models_llama2_build_graph(struct vkllm_context *context, struct vkllm_models_llama2 *model,
                                                   struct vkllm_tensor *input_toks, struct vkllm_graph *graph,
                                                   uint32_t offsets);
/* src/models/vkllm_models_llama2.c:604-816 */
extern vkllm_err_t vkllm_models_llama2_tokenize(struct vkllm_models_llama2 *model, const char *sentence,
                                                struct vkllm_array_token_id **token_ids);

#ifdef __cplusplus
}
#endif
#endif
